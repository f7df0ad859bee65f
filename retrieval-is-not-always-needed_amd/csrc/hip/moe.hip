// MoE MLP block of one decode token (forward_moe of
// arch/mla/deepseek_mla_layer.cu:291-350) for Q2_K experts, in three
// launches instead of the reference's norm, shared gate/up, shared down,
// router, host top-k and per-expert matvec chain:
//   1. router:  a2 = RMSNorm(h, ln2); logits = W_gate_inp a2 (fp32 router,
//               one wave per expert, every workgroup normalizes h itself).
//   2. gate/up: every workgroup takes the top-k of softmax(logits) from the
//               E logits; the rows of the shared FFN and of the k selected
//               experts give G = SiLU(W_g a2) * (W_u a2).  Integer dot
//               products on the 2-bit fields against block floating point
//               digits of a2 (prepared once per workgroup).
//   3. down:    h_i += W_sd[i] . G_sh + sum_j p_j (W_d[e_j][i] . G_j), one
//               wave per row over all its columns (fp32 products weighted
//               by the probabilities, then one reduction: the same terms as
//               the reference's shared matvec + saxpy chain, summed in
//               another order).  G is digitized into LDS per workgroup.
#include <type_traits>

#include "q2k_col.hpp"

namespace {

struct MoeBlkArgs {
    const float* ln2;
    float eps;
    const float* wr;                      // router [E, d] fp32
    const uint8_t *sg, *su, *sd;          // shared gate/up [S, d], down [d, S]
    const uint8_t *wg, *wu, *wd;          // stacked routed experts
    int64_t stride_gu, stride_dn;
    int E, k, d, F, S;
    float* G;                             // ws [S + k F]
    float* a2;                            // ws [d]
    float* logits;                        // ws [E]
    int* ids;                             // ws [k]
    float* probs;                         // ws [k]
    float* h;                             // residual stream [d]
};

constexpr int kMoeMaxD = 2048;    // one 32-value column per lane of a wave

// ---------------------------------------------------------------------------
// 1. router
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void moe_router_kernel(MoeBlkArgs a) {
    __shared__ __align__(16) float s_x[kMoeMaxD];
    __shared__ float red[8];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // the wave's router row first (it does not depend on the norm)
    const int e = blockIdx.x * 4 + wave;
    const float* wrow = a.wr + (int64_t)(e < a.E ? e : 0) * a.d;
    f32x4 w[8];
#pragma unroll
    for (int t = 0; t < 8; t++) {
        const int i = 4 * lane + 256 * t;
        w[t] = i < a.d ? gld((const f32x4*)(wrow + i)) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    f32x4 hv[2], wv[2];
#pragma unroll
    for (int r = 0; r < 2; r++) {
        const int i = 4 * tid + 1024 * r;
        const bool on = i < a.d;
        hv[r] = on ? gld((const f32x4*)(a.h + i)) : f32x4{0.f, 0.f, 0.f, 0.f};
        wv[r] = on ? gld((const f32x4*)(a.ln2 + i)) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    float ss = 0.f;
#pragma unroll
    for (int r = 0; r < 2; r++) {
        ss = fmaf(hv[r].x, hv[r].x, ss);
        ss = fmaf(hv[r].y, hv[r].y, ss);
        ss = fmaf(hv[r].z, hv[r].z, ss);
        ss = fmaf(hv[r].w, hv[r].w, ss);
    }
    const float inv = 1.0f / sqrtf(block_sum4(ss, red, 0) / (float)a.d + a.eps);
#pragma unroll
    for (int r = 0; r < 2; r++) {
        const int i = 4 * tid + 1024 * r;
        if (i < a.d) {
            const f32x4 v = {hv[r].x * inv * wv[r].x, hv[r].y * inv * wv[r].y, hv[r].z * inv * wv[r].z,
                             hv[r].w * inv * wv[r].w};
            *(f32x4*)(s_x + i) = v;
            if (blockIdx.x == 0) gst((f32x4*)(a.a2 + i), v);
        }
    }
    __syncthreads();
    if (e >= a.E) return;
    float acc = 0.f;
#pragma unroll
    for (int t = 0; t < 8; t++) {
        const int i = 4 * lane + 256 * t;
        if (i < a.d) {
            const f32x4 x = *(const f32x4*)(s_x + i);
            acc = fmaf(w[t].x, x.x, acc);
            acc = fmaf(w[t].y, x.y, acc);
            acc = fmaf(w[t].z, x.z, acc);
            acc = fmaf(w[t].w, x.w, acc);
        }
    }
    acc = wave_sum(acc);
    if (lane == 0) gst(a.logits + e, acc);
}

// ---------------------------------------------------------------------------
// 2. gate/up
// ---------------------------------------------------------------------------

// Top-k of softmax(logits) by one wave (E <= 64, lane = expert), the
// reference's selection (deepseek_mla_layer.cu:310-326): it keeps the k
// largest probabilities with strict ">" (of equal values the earlier expert
// stays), in ascending order with equal values later-expert first.  Here k
// rounds each take the largest remaining probability, the lowest expert
// among equal ones, and fill the slots from the top.  The normalizer is
// summed in expert order as the reference's loop does (the exponentials of
// experts >= E are exact zeros).  s_tmp: 64 floats of the wave's own LDS.
__device__ __forceinline__ void topk_wave(const MoeBlkArgs& a, float x, int* s_ids, float* s_pr, float* s_tmp,
                                          bool publish) {
    const int lane = threadIdx.x & 63;
    const float mx = wave_max(x);
    const float ex = lane < a.E ? expf(x - mx) : 0.f;
    s_tmp[lane] = ex;
    if (lane < a.k) s_ids[lane] = -1;
    __builtin_amdgcn_wave_barrier();
    float sum = 0.f;
#pragma unroll
    for (int q = 0; q < 16; q++) {
        const f32x4 v = *(const f32x4*)(s_tmp + 4 * q);
        sum += v.x; sum += v.y; sum += v.z; sum += v.w;
    }
    const float p = ex * (1.0f / sum);
    float pv = lane < a.E ? p : -INFINITY;
    for (int t = 0; t < a.k; t++) {
        const float m = wave_max(pv);
        if (m == -INFINITY) break;                 // fewer than k finite probabilities
        const uint64_t hit = __ballot(pv == m);
        const int win = __builtin_ctzll(hit);      // lowest expert among equal values
        if (lane == win) {
            const int slot = a.k - 1 - t;
            s_ids[slot] = lane;
            s_pr[slot] = p;
            if (publish) {
                gst(a.ids + slot, lane);
                gst(a.probs + slot, p);
            }
            pv = -INFINITY;
        }
    }
    __builtin_amdgcn_wave_barrier();
}

constexpr int kGuRB = 4;   // row pairs per wave per group

struct GuBlk {
    Q2ColQ c[kGuRB][2];     // quad form: d % 128 == 0 keeps every quad on one half page
    int vr[kGuRB];          // virtual row (output index), -1 past the end
    bool ok[kGuRB];         // row has an expert (lane also active)
    bool rowok[kGuRB];
};

__device__ __forceinline__ void gu_issue(const MoeBlkArgs& a, const int* s_ids, int grp, int R, bool active,
                                         GuBlk& b) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < kGuRB; i++) {
        const int vr = grp * kGuRB + i;
        const bool valid = vr < R;
        const uint8_t *wg = a.sg, *wu = a.su;
        int row = vr;
        bool rowok = valid;
        if (vr >= a.S) {
            const int j = min((vr - a.S) / a.F, a.k - 1);
            row = vr - a.S - j * a.F;
            const int e = s_ids[j];
            rowok = valid && e >= 0 && e < a.E;
            const int64_t eo = rowok ? (int64_t)e : 0;
            wg = a.wg + eo * a.stride_gu;
            wu = a.wu + eo * a.stride_gu;
        }
        const bool ok = rowok && active;
        const uint32_t e0 = ok ? (uint32_t)row * (uint32_t)a.d + 32u * lane : 0u;
        q2_colq_issue32(wg, e0, b.c[i][0]);
        q2_colq_issue32(wu, e0, b.c[i][1]);
        b.vr[i] = valid ? vr : -1;
        b.ok[i] = ok;
        b.rowok[i] = rowok;
    }
}

__device__ __forceinline__ void gu_consume(const MoeBlkArgs& a, const DCols<FMT_Q2_K>& xc, const GuBlk& b) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < kGuRB; i++) {
        Q2Col cg, cu;   // the quad exchange runs on every lane, outside the row test
        q2_colq_expand(b.c[i][0], cg);
        q2_colq_expand(b.c[i][1], cu);
        const float g = wave_sum(b.ok[i] ? q2_col(cg, xc) : 0.f);
        const float u = wave_sum(b.ok[i] ? q2_col(cu, xc) : 0.f);
        if (lane == 0 && b.vr[i] >= 0) gst(a.G + b.vr[i], b.rowok[i] ? silu_mul(g, u) : 0.f);
    }
}

// Every wave with routed rows selects the experts itself (no barrier before
// its first weight loads); the loads are in flight while the workgroup
// digitizes a2.
__global__ __launch_bounds__(256) void moe_gate_up_q2_kernel(MoeBlkArgs a) {
    __shared__ PrepLds prep;
    __shared__ int s_ids_w[4][16];
    __shared__ float s_pr_w[4][16];
    __shared__ __align__(16) float s_tmp_w[4][64];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int* s_ids = s_ids_w[wave];
    const bool active = lane < a.d / 32;
    const int R = a.S + a.k * a.F;
    const int ngrp = (R + kGuRB - 1) / kGuRB;
    const int step = gridDim.x * 4;
    int grp = blockIdx.x * 4 + wave;
    const bool publish = blockIdx.x == 0 && wave == 0;
    // a wave whose only row group holds shared-FFN rows needs no expert ids:
    // its weight loads go out at once, during the other waves' logits round
    // trip (wave 0 of workgroup 0 still publishes the selection)
    const bool shared_only = (grp + 1) * kGuRB <= a.S && grp + step >= ngrp && !publish;
    // the logits before a2 (loads complete in issue order: the top-k waits
    // for the logits alone)
    const float lg = !shared_only && lane < a.E ? gld(a.logits + lane) : -INFINITY;
    const PrepSrc src{a.a2, nullptr, a.d, 0.f};
    PrepRaw<4, RINA_PRO_NONE> raw;
    wg_prep_load<4, RINA_PRO_NONE>(src, raw);
    // (one issue site for both: separate copies of the loads leave the
    // load-counter waits after the join counting the wrong loads)
    if (!shared_only) topk_wave(a, lg, s_ids_w[wave], s_pr_w[wave], s_tmp_w[wave], publish);
    GuBlk A, B;
    gu_issue(a, s_ids, grp < ngrp ? grp : 0, R, active && grp < ngrp, A);   // rows < S do not read s_ids
    wg_prep_x<FMT_Q2_K, 4, RINA_PRO_NONE>(src, raw, prep);
    DCols<FMT_Q2_K> xc;
    read_cols<FMT_Q2_K>(prep, lane, active, xc);
    if (grp >= ngrp) return;
    for (;;) {
        if (grp + step < ngrp) {
            gu_issue(a, s_ids, grp + step, R, active, B);
            gu_consume(a, xc, A);
        } else {
            gu_consume(a, xc, A);
            break;
        }
        grp += step;
        if (grp + step < ngrp) {
            gu_issue(a, s_ids, grp + step, R, active, A);
            gu_consume(a, xc, B);
        } else {
            gu_consume(a, xc, B);
            break;
        }
        grp += step;
    }
}

// ---------------------------------------------------------------------------
// 3. down
// ---------------------------------------------------------------------------

// G as block floating point digit columns in LDS: per 32-value column one
// 28-dword record (3 planes x 8 dwords of digits in natural order, the fp32
// sums of the two halves, 2^(e-22), padding).  A 28-dword lane stride keeps
// the 16 lanes of a 16-byte LDS read on distinct banks.
constexpr int kRec = 28;

// Four threads per column (8 values each) digitize G cooperatively.  The
// loads are issued by stage_g_load (before the weight loads, so waiting for
// them does not wait for the weights: loads retire in issue order) and
// consumed by stage_g_digits.
constexpr int kStageRounds = 4;                    // 512 threads x 4 rounds / 4 = 512 columns

// SR rounds of 128 columns (<= kStageRounds)
template <int SR>
struct GStage {
    f32x4 v[SR][2];
};

// Every lane loads (columns past ncol read column 0, which stage_g_digits
// never stores): loads under a branch leave the load-counter waits after it
// waiting for every load in flight.
template <int SR>
__device__ __forceinline__ void stage_g_load(const float* G, int ncol, GStage<SR>& g) {
    const int tid = threadIdx.x, j = tid & 3;
#pragma unroll
    for (int r = 0; r < SR; r++) {
        const int c = (tid >> 2) + 128 * r;
        const f32x4* src = (const f32x4*)(G + 32 * (c < ncol ? c : 0) + 8 * j);
        g.v[r][0] = gld(src);
        g.v[r][1] = gld(src + 1);
    }
}

template <int SR>
__device__ __forceinline__ void stage_g_digits(const GStage<SR>& g, int ncol, uint32_t* rec) {
    const int tid = threadIdx.x, j = tid & 3;
    const int rounds = (ncol + 127) / 128;         // uniform: the group shuffles see full waves
#pragma unroll
    for (int r = 0; r < SR; r++) {
        if (r >= rounds) break;
        const int c = (tid >> 2) + 128 * r;
        const float x[8] = {g.v[r][0].x, g.v[r][0].y, g.v[r][0].z, g.v[r][0].w,
                            g.v[r][1].x, g.v[r][1].y, g.v[r][1].z, g.v[r][1].w};
        float mx = 0.f, hs = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) { mx = fmaxf(mx, fabsf(x[i])); hs += x[i]; }
        mx = grp_max<4>(mx);
        hs += dpp_f<0xB1>(hs);                     // sum of the 16-value half (threads j, j^1)
        int e = 0;
        if (mx > 0.f) (void)frexpf(mx, &e);
        const float up = ldexpf(1.0f, 22 - e);
        uint32_t p[3][2];
#pragma unroll
        for (int t = 0; t < 2; t++)
            digits4(x[4 * t], x[4 * t + 1], x[4 * t + 2], x[4 * t + 3], up, p[0][t], p[1][t], p[2][t]);
        if (c < ncol) {
            uint32_t* rc = rec + c * kRec;
#pragma unroll
            for (int k = 0; k < 3; k++) {
                rc[8 * k + 2 * j] = p[k][0];
                rc[8 * k + 2 * j + 1] = p[k][1];
            }
            if ((j & 1) == 0) rc[24 + (j >> 1)] = __float_as_uint(hs);
            if (j == 0) rc[26] = __float_as_uint(ldexpf(1.0f, e - 22));
        }
    }
}

__device__ __forceinline__ void read_rec(const uint32_t* rc, DCols<FMT_Q2_K>& xc) {
    typedef uint32_t u4 __attribute__((ext_vector_type(4)));
    const u4* r4 = (const u4*)rc;
#pragma unroll
    for (int q = 0; q < 6; q++) {
        const u4 v = r4[q];
        const int k = q >> 1, t = 4 * (q & 1);
        xc.dg[0][k][t] = (int32_t)v.x; xc.dg[0][k][t + 1] = (int32_t)v.y;
        xc.dg[0][k][t + 2] = (int32_t)v.z; xc.dg[0][k][t + 3] = (int32_t)v.w;
    }
    const u4 v = r4[6];
    xc.tt[0][0] = __uint_as_float(v.x);
    xc.tt[0][1] = __uint_as_float(v.y);
    xc.tt[0][2] = 0.f;
    xc.xe[0] = __uint_as_float(v.z);
    xc.xs[0] = 0.f;
}

// Every wave owns one output row.  The row's columns over all its sources
// (the shared chunk columns, then each selected expert's columns, the same
// order as G's 32-value columns) are dealt to the lanes in rounds of 64, so
// no lane idles on a short expert row; each column's product is weighted by
// its source's probability (1 for the shared FFN) and one wave reduction
// gives the row.  The loads go out before the workgroup digitizes G.
// QUAD (shared and expert widths multiples of 128): a quad's four lanes
// hold the four columns of one half page, so each lane loads 8 of its 32
// qs bytes and the quad exchanges them (Q2ColQ) instead of every lane
// loading all 32.
constexpr int kDnRounds = 8;   // columns per lane: (shared + k * ffn) / 32 <= 512

// R: the launch's rounds, ceil(columns / 64) (<= kDnRounds): every lane
// issues R rounds of column loads and ceil(R / 2) rounds of G loads, none
// past the last round (DeepSeek-V2-Lite: 352 columns, 6 rounds, 26 loads
// per wave with the ids instead of 34)
template <bool QUAD, int R>
__global__ __launch_bounds__(512) void moe_down_q2_kernel(MoeBlkArgs a) {
    extern __shared__ __align__(16) uint32_t s_rec[];   // [n / 32][kRec]
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = a.S + a.k * a.F;                 // multiple of 32
    const int ncol = n / 32, fcols = a.F / 32, scols = a.S / 32;
    const int rounds = (ncol + 63) / 64;
    const int i = blockIdx.x * 8 + wave;           // grid covers d rows exactly once
    const bool row_on = i < a.d;
    const int ir = row_on ? i : 0;

    // the selected experts / probabilities and G load together (one round
    // trip); the weight addresses need the expert ids.  Lane j < k holds
    // slot j's expert and probability; a column's slot is read from that
    // lane (ds_bpermute, every lane active) instead of a select chain.
    // (ids first: loads complete in issue order, so the addresses wait for
    // the ids alone)
    const int my_id = lane < a.k ? gld(a.ids + lane) : -1;
    const float my_pr = lane < a.k ? gld(a.probs + lane) : 0.f;
    GStage<(R + 1) / 2> gs;                        // ncol <= 64 R: ceil(R / 2) rounds of 128
    stage_g_load(a.G, ncol, gs);
    // floor(t / fcols) for 0 <= t < 2^16 / 128: t * ceil(2^16 / fcols) >> 16,
    // then one correction step each way
    const uint32_t magic = (65536u + (uint32_t)fcols - 1u) / (uint32_t)fcols;
    typename std::conditional<QUAD, Q2ColQ, Q2Col>::type c[R];
    float wt[R];
    int col[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int cc = 64 * r + lane;
        const int t = cc - scols;                  // routed column index (negative: a shared column)
        const int tt = t < 0 ? 0 : t;
        int j = (int)(((uint32_t)tt * magic) >> 16);
        j -= j * fcols > tt;
        j += (j + 1) * fcols <= tt;
        j = j < a.k ? j : a.k - 1;
        const int e = __shfl(my_id, j);
        const float pj = __shfl(my_pr, j);
        const uint8_t* w = a.sd;
        uint32_t e0 = 0;
        float f = 0.f;
        if (r < rounds && row_on && cc < ncol) {
            if (cc < scols) {
                e0 = (uint32_t)ir * (uint32_t)a.S + 32u * cc;
                f = 1.0f;
            } else if (e >= 0 && e < a.E) {
                w = a.wd + (int64_t)e * a.stride_dn;
                e0 = (uint32_t)ir * (uint32_t)a.F + 32u * (uint32_t)(t - j * fcols);
                f = pj;
            }
        }
        wt[r] = f;
        col[r] = cc < ncol ? cc : 0;
        if constexpr (QUAD) q2_colq_issue32(w, e0, c[r]);
        else q2_col_issue32(w, e0, c[r]);
    }
    stage_g_digits(gs, ncol, s_rec);
    __syncthreads();
    if (!row_on) return;

    float acc = 0.f;
#pragma unroll
    for (int r = 0; r < R; r++) {
        if (r >= rounds) break;                    // wave-uniform (rounds == R)
        Q2Col cx;
        if constexpr (QUAD) q2_colq_expand(c[r], cx);   // every lane of the quad takes part
        else cx = c[r];
        if (wt[r] != 0.f) {
            DCols<FMT_Q2_K> xc;
            read_rec(s_rec + col[r] * kRec, xc);
            acc = fmaf(wt[r], q2_col(cx, xc), acc);
        }
    }
    acc = wave_sum(acc);
    if (lane == 0) gst(a.h + i, gld(a.h + i) + acc);
}

}  // namespace

extern "C" size_t rina_hip_moe_block_workspace(int d, int n_experts, int k, int ffn, int shared_ffn) {
    if (d < 1 || n_experts < 1 || k < 1 || ffn < 1 || shared_ffn < 1) return 0;
    return ((size_t)shared_ffn + (size_t)k * ffn + d + n_experts + 2 * (size_t)k + 4) * sizeof(float);
}

extern "C" int rina_hip_moe_block(float* h, const float* ln2, float eps, const void* gate_inp, int qt_gate_inp,
                                  const void* gate_sh, const void* up_sh, const void* down_sh, int shared_ffn,
                                  const void* gate_exps, const void* up_exps, const void* down_exps, int qt,
                                  int64_t stride_gate_up, int64_t stride_down, int n_experts, int k, int d, int ffn,
                                  void* workspace, size_t ws_bytes, void* stream) {
    if (!h || !ln2 || !gate_inp || !gate_sh || !up_sh || !down_sh || !gate_exps || !up_exps || !down_exps ||
        n_experts < 1 || k < 1 || k > n_experts || d < 1 || ffn < 1 || shared_ffn < 1)
        return RINA_ERR_ARG;
    if (qt != RINA_QT_GGML_Q2_K || qt_gate_inp != RINA_QT_FP32) return RINA_ERR_QTYPE;
    const int S = shared_ffn, F = ffn;
    if (d % 128 || d > kMoeMaxD || F % 32 || F > kMoeMaxD || S % 32 || n_experts > 64 || k > 16) return RINA_ERR_SHAPE;
    const int n = S + k * F;
    const size_t lds = (size_t)(n / 32) * kRec * sizeof(uint32_t);
    if (lds > 64 * 1024 || n > 16384) return RINA_ERR_SHAPE;
    if (((uintptr_t)h | (uintptr_t)ln2 | (uintptr_t)gate_inp | (uintptr_t)workspace) % 16 ||
        ((uintptr_t)gate_sh | (uintptr_t)up_sh | (uintptr_t)down_sh | (uintptr_t)gate_exps | (uintptr_t)up_exps |
         (uintptr_t)down_exps) % 4 || stride_gate_up % 4 || stride_down % 4)
        return RINA_ERR_SHAPE;
    if (!workspace || ws_bytes < rina_hip_moe_block_workspace(d, n_experts, k, F, S)) return RINA_ERR_WORKSPACE;
    MoeBlkArgs a{};
    a.ln2 = ln2; a.eps = eps;
    a.wr = (const float*)gate_inp;
    a.sg = (const uint8_t*)gate_sh; a.su = (const uint8_t*)up_sh; a.sd = (const uint8_t*)down_sh;
    a.wg = (const uint8_t*)gate_exps; a.wu = (const uint8_t*)up_exps; a.wd = (const uint8_t*)down_exps;
    a.stride_gu = stride_gate_up; a.stride_dn = stride_down;
    a.E = n_experts; a.k = k; a.d = d; a.F = F; a.S = S;
    a.G = (float*)workspace;
    a.a2 = a.G + n;                    // n % 32 == 0: stays 16-byte aligned
    a.logits = a.a2 + d;
    a.ids = (int*)(a.logits + n_experts);
    a.probs = (float*)(a.ids + k);
    a.h = h;
    hipStream_t st = as_stream(stream);
    hipLaunchKernelGGL(moe_router_kernel, dim3((n_experts + 3) / 4), dim3(256), 0, st, a);
    RINA_LAUNCH_CHECK();
    const int cus = rina_num_cus();
    const int ngrp = (n + kGuRB - 1) / kGuRB;
    // up to 3 workgroups per CU (DeepSeek-V2-Lite: 704, one row group per
    // wave; a cap of 2 per CU measured 0.3 us slower per layer)
    int g1 = (ngrp + 3) / 4;
    if (g1 > cus * 3) g1 = cus * 3;
    hipLaunchKernelGGL(moe_gate_up_q2_kernel, dim3(g1), dim3(256), 0, st, a);
    RINA_LAUNCH_CHECK();
    // quad column loads when every source's columns come in whole half pages;
    // one instantiation per round count (n <= 16384: at most kDnRounds)
    {
        const bool quad = S % 128 == 0 && F % 128 == 0;
        const int rounds = (n / 32 + 63) / 64;
        const dim3 g3((d + 7) / 8);
#define DN(R)                                                                             \
    do {                                                                                  \
        if (quad) hipLaunchKernelGGL((moe_down_q2_kernel<true, R>), g3, dim3(512), lds, st, a);   \
        else hipLaunchKernelGGL((moe_down_q2_kernel<false, R>), g3, dim3(512), lds, st, a);       \
    } while (0)
        switch (rounds) {
            case 1: DN(1); break;
            case 2: DN(2); break;
            case 3: DN(3); break;
            case 4: DN(4); break;
            case 5: DN(5); break;
            case 6: DN(6); break;
            case 7: DN(7); break;
            default: DN(8); break;
        }
#undef DN
    }
    RINA_LAUNCH_CHECK();
    return RINA_OK;
}
