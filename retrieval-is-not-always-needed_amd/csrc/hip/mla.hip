// DeepSeek MLA decode attention over a latent KV cache, and the MoE router
// and expert FFN (arch/mla/deepseek_mla_layer.cu:171-350), for gfx950.
//
// Attention math (the reference's intended decode semantics, as the CPU
// oracle restates it in expanded form): per head h,
//   q = [q_nope_h | RoPE(q_rope_h)],  K_j = [W_kb_h c_j | RoPE(k_pe_j)],
//   V_j = W_vb_h c_j,  c_j = RMSNorm(c_kv_j) * k_norm,  scale 1/sqrt(nope+rope).
// This build caches the latent record [c_j | RoPE(k_pe_j)] (dc + rope floats
// per position, 2304 B at the DeepSeek-V2-Lite shape, instead of 16 KB of
// expanded K/V) and folds W_kb into the query and W_vb after the softmax:
//   q_lat_h = W_kb_h^T q_nope_h,  s_j = (q_lat_h . c_j + q_rope_h . kpe_j) scale,
//   o_h = W_vb_h (sum_j p_j c_j).
// Short contexts: one launch (mla_fused_kernel).  Longer ones at the
// DeepSeek-V2 shape: two launches, mla_chunk_kernel (per chunk of positions
// and head: q_lat and the chunk's softmax partial in latent space) and
// mla_combine_kernel (chunk merge and W_vb per head).  Other shapes: three launches,
// prep (q_lat, rotated q_rope, latent append at pos0), split (chunk
// partials over positions, one workgroup per chunk and head), out (chunk
// merge and W_vb per head).
//
// MoE: device top-k (no host round trip), a gathered SiLU*up matvec over the
// selected experts, and the down projection that accumulates the experts in
// the reference's ascending order onto the shared-expert output and adds the
// residual.
#include <algorithm>
#include <vector>
#include "rina_common.hpp"

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

// 16 consecutive values [e0, e0+16) of a weight stream in flat element
// order (e0 % 16 == 0): Q2_K (ops/linear.cu:322-338 indexing), Q4_0 / Q4_0F
// (half a block) or fp32.
__device__ __forceinline__ void load_unit16(const uint8_t* w, int qt, int64_t e0, float (&v)[16]) {
    if (qt == RINA_QT_GGML_Q2_K) {
        const uint8_t* bp = w + (e0 >> 8) * 84;
        const int inb = (int)(e0 & 255);
        const int page = inb >> 7, g = (inb >> 5) & 3, h2 = (inb >> 4) & 1;
        const uint32_t dd = gld((const uint32_t*)(bp + 80));
        const uint32_t scb = gld(bp + 8 * page + 2 * g + h2);
        const float dl = f16_to_f32(dd & 0xFFFF) * (float)(scb & 0xF);
        const float ml = f16_to_f32(dd >> 16) * (float)(scb >> 4);
        const uint32_t* qp = (const uint32_t*)(bp + 16 + 32 * page + 16 * h2);
#pragma unroll
        for (int d = 0; d < 4; d++) {
            const uint32_t q = gld(qp + d) >> (2 * g);
#pragma unroll
            for (int b = 0; b < 4; b++) v[4 * d + b] = fmaf(dl, (float)((q >> (8 * b)) & 3), -ml);
        }
    } else if (qt == RINA_QT_Q4_0 || qt == RINA_QT_Q4_0F) {
        const int bb = qt == RINA_QT_Q4_0 ? 18 : 20, so = qt == RINA_QT_Q4_0 ? 2 : 4;
        const uint8_t* bp = w + (e0 >> 5) * bb;
        const int half = (int)((e0 >> 4) & 1);
        float sc;
        if (qt == RINA_QT_Q4_0) sc = f16_to_f32(gld((const uint16_t*)bp));
        else sc = __uint_as_float(gld((const uint32_t*)bp));
        const uint8_t* np = bp + so + 8 * half;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint32_t byte = gld(np + j);
            v[2 * j] = (float)((int)(byte & 0xF) - 7) * sc;
            v[2 * j + 1] = (float)((int)(byte >> 4) - 7) * sc;
        }
    } else {
        const f32x4* p = (const f32x4*)((const float*)w + e0);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const f32x4 x = gld(p + i);
            v[4 * i] = x.x; v[4 * i + 1] = x.y; v[4 * i + 2] = x.z; v[4 * i + 3] = x.w;
        }
    }
}

// dot of row `row` of an [N, K] weight (flat element order) with x (LDS),
// lanes over 16-value units; result in every lane
__device__ __forceinline__ float row_dot(const uint8_t* w, int qt, int64_t row, int K, const float* x, int lane) {
    float acc = 0.f;
    for (int u = lane; u < K / 16; u += 64) {
        float v[16];
        load_unit16(w, qt, row * K + 16 * u, v);
#pragma unroll
        for (int i = 0; i < 16; i++) acc = fmaf(v[i], x[16 * u + i], acc);
    }
    return wave_sum(acc);
}

// N row dots at once (loads of all N rows issued before the FMAs):
// out[r] = W_r[row_r] . x_r, rows of K values in flat element order.
template <int N>
__device__ __forceinline__ void rows_dot(const uint8_t* const (&w)[N], int qt, const int64_t (&row)[N], int K,
                                         const float* const (&x)[N], int lane, float (&out)[N]) {
    float acc[N];
#pragma unroll
    for (int r = 0; r < N; r++) acc[r] = 0.f;
    for (int u = lane; u < K / 16; u += 64) {
        float v[N][16];
#pragma unroll
        for (int r = 0; r < N; r++) load_unit16(w[r], qt, row[r] * K + 16 * u, v[r]);
#pragma unroll
        for (int r = 0; r < N; r++) {
            // 16-byte LDS reads (x 16-byte aligned): scalar reads of a
            // 16-float slice per lane conflict 16 ways across the banks
            const f32x4* xr = (const f32x4*)(x[r] + 16 * u);
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const f32x4 xv = xr[q];
                acc[r] = fmaf(v[r][4 * q], xv.x, acc[r]);
                acc[r] = fmaf(v[r][4 * q + 1], xv.y, acc[r]);
                acc[r] = fmaf(v[r][4 * q + 2], xv.z, acc[r]);
                acc[r] = fmaf(v[r][4 * q + 3], xv.w, acc[r]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < N; r++) out[r] = wave_sum(acc[r]);
}

struct MlaArgs {
    const float* q;        // [H*(nope+rope)]: [H*nope | H*rope]
    const float* kva;      // [dc+rope]: [c_kv | k_pe], raw
    const float* k_norm;   // [dc]
    float eps;
    const float* rc;       // RoPE tables [max_seq][rope/2] (NULL: none)
    const float* rs;
    const uint8_t* wkvb;   // [H*(nope+v), dc]
    int qt;
    float* cache;          // [max_seq][dc+rope] latent records
    float* out;            // [H*v]
    float* ws_q;           // [H][dc+rope]: q_lat | rotated q_rope
    float* ws_m;           // [nchunk][H]
    float* ws_l;
    float* ws_o;           // [nchunk][H][dc]
    int H, nope, rope, v, dc, start_pos, max_seq, chunk;
    int nslot;             // > 0: chunk workgroups; chunk length from the position count (chunk_of)
    const int* d_pos;
    float scale;
};

constexpr int kSplitWaves = 8;         // waves per split workgroup
constexpr int kMlaChunk = 8 * kSplitWaves;   // positions per split block (8 per wave)
constexpr int kMlaMaxChunks = 64;      // chunk partials the out kernel merges (host: chunk length adapts)
constexpr int kPrepRows = 4;           // W_kb rows per prep thread: nope <= 4 * 256 / (dc / 64)
constexpr int kMaxRecLanes = 10;       // record floats per lane: dc + rope <= 640
constexpr int kMaxOutLanes = 8;        // latent dims per lane: dc <= 512

// positions per chunk when L positions are dealt to nslot chunk
// workgroups in whole units of gran positions: as few units per chunk as
// fill the slots (the merging kernel derives the same chunks)
__device__ __forceinline__ int dyn_chunk(int L, int nslot, int gran) {
    const int nt = (L + gran - 1) / gran;
    return gran * ((nt + nslot - 1) / nslot);
}

// a.nslot > 0: chunks follow the position count (a.chunk is the unit);
// else a.chunk positions per chunk
__device__ __forceinline__ int chunk_of(const MlaArgs& a, int L) {
    return a.nslot > 0 ? dyn_chunk(L, a.nslot, a.chunk) : a.chunk;
}

// NeoX rotation of pair (i, i+rope/2) at table row pos, reference fma form
__device__ __forceinline__ void rope_pair(float x0, float x1, float c, float s, float& o0, float& o1) {
    o0 = fmaf(x0, c, -(x1 * s));
    o1 = fmaf(x0, s, x1 * c);
}

// grid H + 1: workgroup h < H builds q_lat_h and the rotated q_rope_h;
// workgroup H appends the latent record of position pos0.
__global__ __launch_bounds__(256) void mla_prep_kernel(MlaArgs a) {
    __shared__ __align__(16) float s_q[512];
    __shared__ float s_part[4096];
    __shared__ float s_red[4];
    const int tid = threadIdx.x;
    const int pos = read_pos(a.start_pos, a.d_pos);
    if (pos < 0 || pos >= a.max_seq) return;
    const int R = a.dc + a.rope, hr = a.rope / 2;
    if (blockIdx.x == (unsigned)a.H) {
        if (blockIdx.y) return;
        // the record [RMSNorm(c_kv) * k_norm | RoPE(k_pe)]: every input is
        // loaded up front (one memory round trip), dc <= 512, rope / 2 <= 256
        const int k0 = tid < a.dc ? tid : 0, k1 = tid + 256 < a.dc ? tid + 256 : 0, jr = tid < hr ? tid : 0;
        const float x0 = gld(a.kva + k0), x1 = gld(a.kva + k1);
        const float n0 = gld(a.k_norm + k0), n1 = gld(a.k_norm + k1);
        float p0 = gld(a.kva + a.dc + jr), p1 = gld(a.kva + a.dc + (hr ? jr + hr : 0));
        const float* tc = a.rc ? a.rc : a.kva;
        const float* ts = a.rs ? a.rs : a.kva;
        const float cc = gld(tc + (a.rc ? (int64_t)pos * hr + jr : 0)), sn = gld(ts + (a.rs ? (int64_t)pos * hr + jr : 0));
        float ss = (tid < a.dc ? x0 * x0 : 0.f);
        ss = fmaf(tid + 256 < a.dc ? x1 : 0.f, tid + 256 < a.dc ? x1 : 0.f, ss);
        ss = wave_sum(ss);
        if ((tid & 63) == 0) s_red[tid >> 6] = ss;
        __syncthreads();
        const float inv = 1.0f / sqrtf(((s_red[0] + s_red[1]) + (s_red[2] + s_red[3])) / (float)a.dc + a.eps);
        float* rec = a.cache + (int64_t)pos * R;
        if (tid < a.dc) gst(rec + tid, x0 * inv * n0);
        if (tid + 256 < a.dc) gst(rec + tid + 256, x1 * inv * n1);
        if (tid < hr) {
            if (a.rc) rope_pair(p0, p1, cc, sn, p0, p1);
            gst(rec + a.dc + tid, p0);
            gst(rec + a.dc + tid + hr, p1);
        }
        return;
    }
    const int h = blockIdx.x;
    float* qo = a.ws_q + (int64_t)h * R;
    // q_lat[k] = sum_i q_nope[i] W[h*nope + i][k] for this workgroup's column
    // quarter: thread = (row slice, 16-column unit).  The thread's weight
    // units (at most kPrepRows rows; the host checks) are loaded before
    // q_nope is staged, so one memory round trip covers both.
    const int ncu = a.dc / 64;
    const int RS = 256 / ncu;
    const int cu = blockIdx.y * ncu + tid % ncu, rsl = tid / ncu;
    float w[kPrepRows][16];
#pragma unroll
    for (int j = 0; j < kPrepRows; j++) {
        const int i = rsl + j * RS < a.nope ? rsl + j * RS : a.nope - 1;
        load_unit16(a.wkvb, a.qt, ((int64_t)h * a.nope + i) * a.dc + 16 * cu, w[j]);
    }
    stage_lds(s_q, a.q + (int64_t)h * a.nope, a.nope);
    for (int j = tid; j < hr && blockIdx.y == 0; j += 256) {
        const float* qr = a.q + (int64_t)a.H * a.nope + (int64_t)h * a.rope;
        float x0 = gld(qr + j), x1 = gld(qr + j + hr);
        if (a.rc) rope_pair(x0, x1, gld(a.rc + (int64_t)pos * hr + j), gld(a.rs + (int64_t)pos * hr + j), x0, x1);
        gst(qo + a.dc + j, x0);
        gst(qo + a.dc + j + hr, x1);
    }
    __syncthreads();
    float acc[16];
#pragma unroll
    for (int j = 0; j < 16; j++) acc[j] = 0.f;
#pragma unroll
    for (int jr = 0; jr < kPrepRows; jr++) {
        const int i = rsl + jr * RS;
        const float qi = i < a.nope ? s_q[i] : 0.f;
#pragma unroll
        for (int j = 0; j < 16; j++) acc[j] = fmaf(qi, w[jr][j], acc[j]);
    }
    const int cw = a.dc / 4;                      // columns of this workgroup
#pragma unroll
    for (int j = 0; j < 16; j++) s_part[rsl * cw + 16 * (tid % ncu) + j] = acc[j];
    __syncthreads();
    for (int k = tid; k < cw; k += 256) {
        float t = 0.f;
        for (int r = 0; r < RS; r++) t += s_part[r * cw + k];
        gst(qo + blockIdx.y * cw + k, t);
    }
}

// grid (nchunk, H): the workgroup walks its chunk (a.chunk positions, a
// multiple of kMlaChunk) in blocks of kMlaChunk; each wave takes 8 positions
// of a block (loads issued together), lanes cover the record's dims.  Per
// block: the wave's 8 scores first (independent dot products and
// reductions), then one softmax update (maximum, rescale, weights; base-2
// units).  Waves merged in LDS, chunk partials (m, l, sum p c) written.
__global__ __launch_bounds__(64 * kSplitWaves) void mla_split_kernel(MlaArgs a) {
    __shared__ float s_o[kSplitWaves][512];
    __shared__ float s_m[kSplitWaves], s_l[kSplitWaves];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int pos0 = read_pos(a.start_pos, a.d_pos);
    if (pos0 < 0 || pos0 >= a.max_seq) return;
    const int L = pos0 + 1, c = blockIdx.x, h = blockIdx.y;
    const int jc = c * a.chunk;
    if (jc >= L) return;
    const int jend = min(jc + a.chunk, L);
    const int R = a.dc + a.rope;
    const float* qh = a.ws_q + (int64_t)h * R;
    float qv[kMaxRecLanes];
#pragma unroll
    for (int j = 0; j < kMaxRecLanes; j++) qv[j] = (lane + 64 * j < R) ? gld(qh + lane + 64 * j) : 0.f;
    const float sc2 = a.scale * 1.44269504088896341f;
    constexpr int PW = kMlaChunk / kSplitWaves;
    float m = -INFINITY, l = 0.f, o[kMaxOutLanes];
#pragma unroll
    for (int j = 0; j < kMaxOutLanes; j++) o[j] = 0.f;
    for (int j0 = jc; j0 < jend; j0 += kMlaChunk) {
        const int ncv = min(kMlaChunk, jend - j0);
        // this wave's positions: j0 + wave + kSplitWaves i (past the block
        // end: its first position, masked below)
        float kv[PW][kMaxRecLanes];
#pragma unroll
        for (int i = 0; i < PW; i++) {
            const int p = wave + kSplitWaves * i;
            const float* rec = a.cache + (int64_t)(j0 + (p < ncv ? p : 0)) * R;
#pragma unroll
            for (int j = 0; j < kMaxRecLanes; j++) kv[i][j] = (lane + 64 * j < R) ? gld(rec + lane + 64 * j) : 0.f;
        }
        float dot[PW];
#pragma unroll
        for (int i = 0; i < PW; i++) {
            float d = 0.f;
#pragma unroll
            for (int j = 0; j < kMaxRecLanes; j++) d = fmaf(qv[j], kv[i][j], d);
            dot[i] = d;
        }
#pragma unroll
        for (int i = 0; i < PW; i++) dot[i] = wave_sum(dot[i]) * sc2;
        float mb = m;
#pragma unroll
        for (int i = 0; i < PW; i++)
            if (wave + kSplitWaves * i < ncv) mb = fmaxf(mb, dot[i]);
        if (mb == -INFINITY) continue;                     // no position of this wave in the block
        const float al = __builtin_amdgcn_exp2f(m - mb);   // 0 while m is -inf
        l *= al;
#pragma unroll
        for (int j = 0; j < kMaxOutLanes; j++) o[j] *= al;
#pragma unroll
        for (int i = 0; i < PW; i++) {
            const float pe = wave + kSplitWaves * i < ncv ? __builtin_amdgcn_exp2f(dot[i] - mb) : 0.f;
            l += pe;
#pragma unroll
            for (int j = 0; j < kMaxOutLanes; j++) o[j] = fmaf(pe, kv[i][j], o[j]);
        }
        m = mb;
    }
#pragma unroll
    for (int j = 0; j < kMaxOutLanes; j++)
        if (lane + 64 * j < a.dc) s_o[wave][lane + 64 * j] = o[j];
    if (lane == 0) { s_m[wave] = m; s_l[wave] = l; }
    __syncthreads();
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kSplitWaves; w++) M = fmaxf(M, s_m[w]);
    float aw[kSplitWaves];
#pragma unroll
    for (int w = 0; w < kSplitWaves; w++) aw[w] = s_m[w] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(s_m[w] - M);
    float* wo = a.ws_o + ((int64_t)c * a.H + h) * a.dc;
    for (int k = tid; k < a.dc; k += 64 * kSplitWaves) {
        float t = 0.f;
#pragma unroll
        for (int w = 0; w < kSplitWaves; w++) t = fmaf(s_o[w][k], aw[w], t);
        gst(wo + k, t);
    }
    if (tid == 0) {
        float lt = 0.f;
#pragma unroll
        for (int w = 0; w < kSplitWaves; w++) lt = fmaf(s_l[w], aw[w], lt);
        gst(a.ws_m + (int64_t)c * a.H + h, M);
        gst(a.ws_l + (int64_t)c * a.H + h, lt);
    }
}

// grid (H, v/16): merge the chunks of head h into o_lat (every workgroup of
// the head repeats this small merge), then 16 rows of out_h = W_vb_h o_lat,
// 4 per wave.  Every load the workgroup needs (its W_vb units, the chunk
// maxima / sums and both latent values of each chunk for this thread) is
// issued at entry: one memory round trip, then LDS work.
__global__ __launch_bounds__(256) void mla_out_kernel(MlaArgs a) {
    __shared__ float s_w[256];
    __shared__ __align__(16) float s_lat[512];
    __shared__ float s_red[8];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int pos0 = read_pos(a.start_pos, a.d_pos);
    if (pos0 < 0 || pos0 >= a.max_seq) return;
    const int nch = pos0 / chunk_of(a, pos0 + 1) + 1;      // <= kMlaMaxChunks
    const int h = blockIdx.x;
    // this wave's 4 rows (v % 4 == 0; rows past v: a clamped row, not stored)
    const int i0 = 16 * blockIdx.y + 4 * wave;
    const bool rows_ok = i0 < a.v;
    const int64_t row0 = (int64_t)a.H * a.nope + (int64_t)h * a.v + (rows_ok ? i0 : 0);
    const int units = a.dc / 16, ul = lane < units ? lane : 0;   // dc <= 1024: one unit per lane
    float wv[4][16];
#pragma unroll
    for (int r = 0; r < 4; r++) load_unit16(a.wkvb, a.qt, (row0 + r) * a.dc + 16 * ul, wv[r]);
    const float mc = tid < nch ? gld(a.ws_m + (int64_t)tid * a.H + h) : -INFINITY;
    const float lc = tid < nch ? gld(a.ws_l + (int64_t)tid * a.H + h) : 0.f;
    const int k0 = tid < a.dc ? tid : 0, k1 = tid + 256 < a.dc ? tid + 256 : 0;
    float v0[kMlaMaxChunks], v1[kMlaMaxChunks];
#pragma unroll
    for (int cc = 0; cc < kMlaMaxChunks; cc++) {
        const float* po = a.ws_o + ((int64_t)(cc < nch ? cc : nch - 1) * a.H + h) * a.dc;
        v0[cc] = gld(po + k0);
        v1[cc] = gld(po + k1);
    }
    const float mw = wave_max(mc);
    if (lane == 0) s_red[wave] = mw;
    __syncthreads();
    const float M = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
    const float w = tid < nch ? __builtin_amdgcn_exp2f(mc - M) : 0.f;   // partial maxima in base-2 units
    s_w[tid] = w;
    const float lw = wave_sum(w * lc);
    __syncthreads();
    if (lane == 0) s_red[4 + wave] = lw;
    __syncthreads();
    const float inv_l = 1.0f / ((s_red[4] + s_red[5]) + (s_red[6] + s_red[7]));
    // o_lat = sum_c w_c O_c / sum_c w_c l_c (weight 0 past nch)
    float acc0 = 0.f, acc1 = 0.f;
#pragma unroll
    for (int cc = 0; cc < kMlaMaxChunks; cc++) {
        acc0 = fmaf(v0[cc], s_w[cc], acc0);
        acc1 = fmaf(v1[cc], s_w[cc], acc1);
    }
    if (tid < a.dc) s_lat[tid] = acc0 * inv_l;
    if (tid + 256 < a.dc) s_lat[tid + 256] = acc1 * inv_l;
    __syncthreads();
    float o4[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        float acc = 0.f;
        if (lane < units) {
            // 16-byte LDS reads of the lane's 16-value slice
            const f32x4* xr = (const f32x4*)(s_lat + 16 * lane);
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const f32x4 xv = xr[q];
                acc = fmaf(wv[r][4 * q], xv.x, acc);
                acc = fmaf(wv[r][4 * q + 1], xv.y, acc);
                acc = fmaf(wv[r][4 * q + 2], xv.z, acc);
                acc = fmaf(wv[r][4 * q + 3], xv.w, acc);
            }
        }
        o4[r] = wave_sum(acc);
    }
    if (rows_ok && lane < 4)
        gst(a.out + (int64_t)h * a.v + i0 + lane, lane == 0 ? o4[0] : lane == 1 ? o4[1] : lane == 2 ? o4[2] : o4[3]);
}

// ---------------------------------------------------------------------------
// The whole attention in one launch (short contexts)
// ---------------------------------------------------------------------------
// grid (H, kFusedY), 1024 threads.  Every workgroup of head h forms q_lat_h
// (W_kb_h^T q_nope_h), the new latent record (kept in LDS; workgroup (0, 0)
// also stores it in the cache), the softmax over the cache in blocks of 64
// positions (4 per wave; the first block's loads go out at kernel entry with
// the weight loads) and o_lat; then it computes its quarter of the W_vb rows.
// The workgroups of a head repeat the attention instead of exchanging
// partials: an exchange inside one launch needs device-scope fences, which
// cost more than the repeated work, and the three-launch path pays a
// dependent launch per stage.  Any position count is computed correctly;
// past one block every further block costs a load round trip, so the host
// uses this kernel below kFusedMaxPos positions.

constexpr int kFusedDc = 512;                 // latent width this kernel is built for
constexpr int kFusedNcu = kFusedDc / 16;      // 16-value units per latent row
constexpr int kFusedRs = 1024 / kFusedNcu;    // row slices of the W_kb contraction
constexpr int kFusedRope = 64;
constexpr int kFusedR = kFusedDc + kFusedRope;   // record floats: 576, 9 per lane
constexpr int kFusedRec = kFusedR / 64;
constexpr int kFusedPw = 4;                   // positions per wave per block
constexpr int kFusedBlock = 16 * kFusedPw;
constexpr int kFusedY = 4;                    // workgroups per head
constexpr int kFusedMaxPos = 256;
constexpr int kChunkTarget = 16;              // chunks of the two-launch path (mla_chunk_kernel)

typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef float f32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));

// The raw bytes of the 16 values [e0, e0 + 16) of a quantized weight stream
// (e0 % 16 == 0), loaded at once and decoded where they are used.
struct RawUnit {
    uint32_t q[4];   // Q2_K: qs bytes; Q4_0F: nibble bytes in q[0..1]; Q4_0: nibble half-words
    uint32_t m;      // Q2_K: d | dmin << 16; Q4_0F: fp32 scale bits; Q4_0: fp16 scale bits
    uint32_t s;      // Q2_K: the 4-bit scale | 4-bit min byte
    int sh;          // Q2_K: the 2-bit field's shift 2g (from the address: no wait on the loads)
};

template <int QT>
__device__ __forceinline__ void raw_issue(RawUnit& u, const uint8_t* w, int64_t e0) {
    if (QT == RINA_QT_GGML_Q2_K) {
        const uint8_t* bp = w + (e0 >> 8) * 84;
        const int inb = (int)(e0 & 255);
        const int page = inb >> 7, g = (inb >> 5) & 3, h2 = (inb >> 4) & 1;
        const u32x4_a4 v = gld((const u32x4_a4*)(bp + 16 + 32 * page + 16 * h2));
        u.q[0] = v.x; u.q[1] = v.y; u.q[2] = v.z; u.q[3] = v.w;
        u.m = gld((const uint32_t*)(bp + 80));
        u.s = gld(bp + 8 * page + 2 * g + h2);
        u.sh = 2 * g;
    } else if (QT == RINA_QT_Q4_0F) {
        const uint8_t* bp = w + (e0 >> 5) * 20;
        const uint32_t* np = (const uint32_t*)(bp + 4 + 8 * ((e0 >> 4) & 1));
        u.q[0] = gld(np); u.q[1] = gld(np + 1);
        u.m = gld((const uint32_t*)bp);
    } else {   // Q4_0: 18-byte blocks, 2-byte aligned
        const uint8_t* bp = w + (e0 >> 5) * 18;
        const uint16_t* np = (const uint16_t*)(bp + 2 + 8 * ((e0 >> 4) & 1));
#pragma unroll
        for (int d = 0; d < 4; d++) u.q[d] = gld(np + d);
        u.m = gld((const uint16_t*)bp);
    }
}

// the 8 nibble bytes of a Q4 unit as two dwords (value 2j: low nibble of
// byte j, value 2j + 1: its high nibble)
template <int QT>
__device__ __forceinline__ void raw_nibbles(const RawUnit& u, uint32_t& d0, uint32_t& d1, float& sc) {
    if (QT == RINA_QT_Q4_0F) {
        d0 = u.q[0]; d1 = u.q[1];
        sc = __uint_as_float(u.m);
    } else {
        d0 = u.q[0] | (u.q[1] << 16); d1 = u.q[2] | (u.q[3] << 16);
        sc = f16_to_f32(u.m);
    }
}

__device__ __forceinline__ float ubyte(uint32_t t, int b) { return (float)((t >> (8 * b)) & 0xFF); }

// acc[j] += c * w_j - (the unit's offset term, gathered in bias): the
// dequantized unit w_j = dl v_j - ml (Q2_K) or sc (n_j - 7) (Q4) scaled by c.
template <int QT>
__device__ __forceinline__ void raw_fold(const RawUnit& u, float c, float (&acc)[16], float& bias) {
    if (QT == RINA_QT_GGML_Q2_K) {
        const float a = c * (f16_to_f32(u.m & 0xFFFF) * (float)(u.s & 0xF));
        bias = fmaf(c, f16_to_f32(u.m >> 16) * (float)(u.s >> 4), bias);
        const int sh = u.sh;
#pragma unroll
        for (int d = 0; d < 4; d++) {
            const uint32_t t = and_opaque(u.q[d] >> sh, 0x03030303u);
#pragma unroll
            for (int b = 0; b < 4; b++) acc[4 * d + b] = fmaf(a, ubyte(t, b), acc[4 * d + b]);
        }
    } else {
        uint32_t dw[2];
        float sc;
        raw_nibbles<QT>(u, dw[0], dw[1], sc);
        const float a = c * sc;
        bias = fmaf(7.0f, a, bias);
#pragma unroll
        for (int d = 0; d < 2; d++) {
            const uint32_t lo = and_opaque(dw[d], 0x0F0F0F0Fu), hi = and_opaque(dw[d] >> 4, 0x0F0F0F0Fu);
#pragma unroll
            for (int b = 0; b < 4; b++) {
                acc[8 * d + 2 * b] = fmaf(a, ubyte(lo, b), acc[8 * d + 2 * b]);
                acc[8 * d + 2 * b + 1] = fmaf(a, ubyte(hi, b), acc[8 * d + 2 * b + 1]);
            }
        }
    }
}

// sum_j w_j x_j over the unit, x: 16 floats in LDS (16-byte aligned)
template <int QT>
__device__ __forceinline__ float raw_dot(const RawUnit& u, const float* x) {
    float xv[16];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const f32x4 t = ((const f32x4*)x)[q];
        xv[4 * q] = t.x; xv[4 * q + 1] = t.y; xv[4 * q + 2] = t.z; xv[4 * q + 3] = t.w;
    }
    float d = 0.f, xs = 0.f;
    if (QT == RINA_QT_GGML_Q2_K) {
        const int sh = u.sh;
#pragma unroll
        for (int dw = 0; dw < 4; dw++) {
            const uint32_t t = and_opaque(u.q[dw] >> sh, 0x03030303u);
#pragma unroll
            for (int b = 0; b < 4; b++) {
                d = fmaf(ubyte(t, b), xv[4 * dw + b], d);
                xs += xv[4 * dw + b];
            }
        }
        const float dl = f16_to_f32(u.m & 0xFFFF) * (float)(u.s & 0xF);
        const float ml = f16_to_f32(u.m >> 16) * (float)(u.s >> 4);
        return fmaf(dl, d, -(ml * xs));
    } else {
        uint32_t dw[2];
        float sc;
        raw_nibbles<QT>(u, dw[0], dw[1], sc);
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const uint32_t lo = and_opaque(dw[k], 0x0F0F0F0Fu), hi = and_opaque(dw[k] >> 4, 0x0F0F0F0Fu);
#pragma unroll
            for (int b = 0; b < 4; b++) {
                d = fmaf(ubyte(lo, b), xv[8 * k + 2 * b], d);
                d = fmaf(ubyte(hi, b), xv[8 * k + 2 * b + 1], d);
                xs += xv[8 * k + 2 * b] + xv[8 * k + 2 * b + 1];
            }
        }
        return sc * fmaf(-7.0f, xs, d);
    }
}

// The cache records of this wave's positions blk + wave + 16 i; lane l
// holds record floats l + 64 j (dword loads: each record line is touched
// once per wave).  Every load is issued (positions >= pos0 read record 0 and
// are never used): branches around loads make the compiler wait for every
// earlier load at the join.
__device__ __forceinline__ void fused_load_block(float (&kv)[kFusedPw][kFusedRec], const float* cache, int blk,
                                                 int wave, int pos0, int lane) {
#pragma unroll
    for (int i = 0; i < kFusedPw; i++) {
        const int p = blk + wave + 16 * i;
        const float* rec = cache + (int64_t)(p < pos0 ? p : 0) * kFusedR + lane;
#pragma unroll
        for (int j = 0; j < kFusedRec; j++) kv[i][j] = gld(rec + 64 * j);
    }
}

template <int QT>
__global__ __launch_bounds__(1024) void mla_fused_kernel(MlaArgs a) {
    __shared__ __align__(16) float s_part[kFusedRs * kFusedDc];   // W_kb partials, then wave partials
    __shared__ __align__(16) float s_q[kFusedR];                  // q_lat | rotated q_rope
    __shared__ __align__(16) float s_rec[kFusedR];                // the new record
    __shared__ __align__(16) float s_lat[kFusedDc];
    __shared__ float s_qn[128];
    __shared__ float s_m[16], s_l[16], s_red[4];
    // the wave index as a uniform value: position tests become scalar branches
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int pos0 = read_pos(a.start_pos, a.d_pos);
    if (pos0 < 0 || pos0 >= a.max_seq) return;
    const int h = blockIdx.x, y = blockIdx.y;
    const int R = kFusedR, hr = kFusedRope / 2, L = pos0 + 1;
    const int cu = tid & (kFusedNcu - 1), rs = tid / kFusedNcu;
    // the small loads first (q_nope, q_rope, k_pe, RoPE tables, c_kv,
    // k_norm): waiting for them then leaves the weight and cache loads,
    // issued after, in flight
    const int ti = tid < hr ? tid : 0;
    const float* qr = a.q + (int64_t)a.H * a.nope + (int64_t)h * kFusedRope;
    const float qn = gld(a.q + (int64_t)h * a.nope + (tid < a.nope ? tid : 0));
    float x0 = gld(qr + ti), x1 = gld(qr + ti + hr);
    float k0 = gld(a.kva + kFusedDc + ti), k1 = gld(a.kva + kFusedDc + ti + hr);
    float rc = 1.f, rsn = 0.f;
    if (a.rc) { rc = gld(a.rc + (int64_t)pos0 * hr + ti); rsn = gld(a.rs + (int64_t)pos0 * hr + ti); }
    const float cx = gld(a.kva + (tid & (kFusedDc - 1))), cn = gld(a.k_norm + (tid & (kFusedDc - 1)));
    const float cx2 = gld(a.kva + (tid & 255) + 256);
    __builtin_amdgcn_sched_barrier(0);   // keep the issue order: small loads, weights, cache
    // weight loads: W_kb_h rows rs + 32 r (column unit cu; rows past nope
    // re-read row 0 with coefficient 0), one W_vb_h row
    RawUnit wk[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int i = rs + kFusedRs * r;
        raw_issue<QT>(wk[r], a.wkvb, ((int64_t)h * a.nope + (i < a.nope ? i : 0)) * kFusedDc + 16 * cu);
    }
    const int vq = (a.v + kFusedY - 1) / kFusedY;
    const int vrow = y * vq + rs;
    const bool vok = rs < vq && vrow < a.v;
    RawUnit wv;
    raw_issue<QT>(wv, a.wkvb, ((int64_t)a.H * a.nope + (int64_t)h * a.v + (vok ? vrow : 0)) * kFusedDc + 16 * cu);
    __builtin_amdgcn_sched_barrier(0);
    float kv[kFusedPw][kFusedRec];
    fused_load_block(kv, a.cache, 0, wave, pos0, lane);
    __builtin_amdgcn_sched_barrier(0);
    // q_nope, rotated q_rope, the record's RoPE half and norm partials (the
    // sum order of mla_prep_kernel: threads 0..255, k = tid, tid + 256)
    if (tid < a.nope) s_qn[tid] = qn;
    if (tid < hr) {
        if (a.rc) {
            rope_pair(x0, x1, rc, rsn, x0, x1);
            rope_pair(k0, k1, rc, rsn, k0, k1);
        }
        s_q[kFusedDc + tid] = x0;
        s_q[kFusedDc + tid + hr] = x1;
        s_rec[kFusedDc + tid] = k0;
        s_rec[kFusedDc + tid + hr] = k1;
        if (h == 0 && y == 0) {
            float* rec = a.cache + (int64_t)pos0 * R;
            gst(rec + kFusedDc + tid, k0);
            gst(rec + kFusedDc + tid + hr, k1);
        }
    }
    if (tid < 256) {
        const float ss = wave_sum(fmaf(cx2, cx2, fmaf(cx, cx, 0.f)));
        if (lane == 0) s_red[wave] = ss;
    }
    __syncthreads();
    // q_lat partials of this thread's rows, then the normalized record
    {
        float acc[16], bias = 0.f;
#pragma unroll
        for (int j = 0; j < 16; j++) acc[j] = 0.f;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int i = rs + kFusedRs * r;
            raw_fold<QT>(wk[r], i < a.nope ? s_qn[i] : 0.f, acc, bias);
        }
        f32x4* dst = (f32x4*)(s_part + rs * kFusedDc + 16 * cu);
#pragma unroll
        for (int q = 0; q < 4; q++)
            dst[q] = f32x4{acc[4 * q] - bias, acc[4 * q + 1] - bias, acc[4 * q + 2] - bias, acc[4 * q + 3] - bias};
    }
    if (tid < kFusedDc) {
        const float inv = 1.0f / sqrtf(((s_red[0] + s_red[1]) + (s_red[2] + s_red[3])) / (float)kFusedDc + a.eps);
        const float v = cx * inv * cn;
        s_rec[tid] = v;
        if (h == 0 && y == 0) gst(a.cache + (int64_t)pos0 * R + tid, v);
    }
    __syncthreads();
    if (tid < kFusedDc) {
        float t = 0.f;
#pragma unroll 8
        for (int r = 0; r < kFusedRs; r++) t += s_part[r * kFusedDc + tid];
        s_q[tid] = t;
    }
    __syncthreads();
    // softmax over the cache, per wave: scores of a block first, then one
    // rescale of the running sums per block.  Scores are kept in base-2
    // units (log2 e folded into the scale) for the hardware exp2.
    const int wu = wave;
    float qv[kFusedRec];
#pragma unroll
    for (int j = 0; j < kFusedRec; j++) qv[j] = s_q[lane + 64 * j];
    const float sc2 = a.scale * 1.44269504088896341f;
    float m = -INFINITY, l = 0.f, o[kFusedDc / 64];
#pragma unroll
    for (int j = 0; j < kFusedDc / 64; j++) o[j] = 0.f;
    for (int blk = 0; blk < L; blk += kFusedBlock) {
        if (blk) fused_load_block(kv, a.cache, blk, wu, pos0, lane);
        float s[kFusedPw];
        float mb = -INFINITY;
#pragma unroll
        for (int i = 0; i < kFusedPw; i++) {
            const int p = blk + wu + 16 * i;
            s[i] = -INFINITY;
            if (p < L) {
                if (p == pos0) {
#pragma unroll
                    for (int j = 0; j < kFusedRec; j++) kv[i][j] = s_rec[lane + 64 * j];
                }
                float dot = 0.f;
#pragma unroll
                for (int j = 0; j < kFusedRec; j++) dot = fmaf(qv[j], kv[i][j], dot);
                s[i] = wave_sum(dot) * sc2;
                mb = fmaxf(mb, s[i]);
            }
        }
        if (mb == -INFINITY) continue;
        const float mn = fmaxf(m, mb), al = __builtin_amdgcn_exp2f(m - mn);
        l *= al;
#pragma unroll
        for (int j = 0; j < kFusedDc / 64; j++) o[j] *= al;
        m = mn;
#pragma unroll
        for (int i = 0; i < kFusedPw; i++) {
            if (s[i] == -INFINITY) continue;
            const float pe = __builtin_amdgcn_exp2f(s[i] - mn);
            l += pe;
#pragma unroll
            for (int j = 0; j < kFusedDc / 64; j++) o[j] = fmaf(pe, kv[i][j], o[j]);
        }
    }
#pragma unroll
    for (int j = 0; j < kFusedDc / 64; j++) s_part[wu * kFusedDc + lane + 64 * j] = o[j];
    if (lane == 0) { s_m[wu] = m; s_l[wu] = l; }
    __syncthreads();
    // merge of the 16 waves (every merging thread forms the wave weights)
    if (tid < kFusedDc) {
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < 16; w++) M = fmaxf(M, s_m[w]);
        float t = 0.f, den = 0.f;
#pragma unroll
        for (int w = 0; w < 16; w++) {
            const float mw = s_m[w];
            const float aw = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - M);
            den = fmaf(aw, s_l[w], den);
            t = fmaf(aw, s_part[w * kFusedDc + tid], t);
        }
        s_lat[tid] = t * (1.0f / den);
    }
    __syncthreads();
    // W_vb row vrow: the 32 units of the row are lanes 0..31 or 32..63
    float pv = raw_dot<QT>(wv, s_lat + 16 * cu);
    pv = sum16(pv);
    pv += dpp_rows<0x142, 0xA>(pv);   // row_bcast:15: lane 31 = lanes 0..31, lane 63 = lanes 32..63
    if (vok && (lane & 31) == 31) gst(a.out + (int64_t)h * a.v + vrow, pv);
}

// ---------------------------------------------------------------------------
// Longer contexts at the DeepSeek-V2 shape: two launches.
// mla_chunk_kernel, grid (chunks padded to the 8 XCDs, H), 1024 threads:
// every workgroup forms q_lat_h and the current record as mla_fused_kernel
// does, scores only its chunk of positions (blocks of 64, 4 per wave) and
// merges its 16 waves into the unnormalized latent partial
// sum_p 2^(s_p - M_c) c_p.  It writes (M_c, l_c, partial) per chunk;
// mla_combine_kernel merges the chunks of each head and applies W_vb_h once
// (applying it per chunk cost every chunk workgroup 1.6 us and the
// registers that made the kernel spill).  The workgroup whose chunk holds
// pos0 of head 0 stores the record.
// The grid has nslot = min(kChunkTarget, max_pos / 64) chunk slots per head;
// the chunk length is derived from the position count at run time (whole
// 64-position blocks, as few per chunk as fill the slots), so a replayed
// graph uses all its slots at every position.  Every chunk workgroup repeats
// q_lat, and the heads of a chunk each stream its records, so 16 chunks per
// head measured best (fewer leave CUs idle, more repeat the fixed work).
// ---------------------------------------------------------------------------
template <int QT>
__global__ __launch_bounds__(1024) void mla_chunk_kernel(MlaArgs a) {
    __shared__ __align__(16) float s_part[kFusedRs * kFusedDc];   // W_kb partials, then wave partials
    __shared__ __align__(16) float s_q[kFusedR];                  // q_lat | rotated q_rope
    __shared__ __align__(16) float s_rec[kFusedR];                // the new record
    __shared__ float s_qn[128];
    __shared__ float s_m[16], s_l[16], s_red[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int pos0 = read_pos(a.start_pos, a.d_pos);
    if (pos0 < 0 || pos0 >= a.max_seq) return;
    const int c = blockIdx.x, h = blockIdx.y;
    const int L = pos0 + 1, chunk = chunk_of(a, L), jc = c * chunk;
    if (jc >= L) return;                                          // padding / chunks past pos0
    const int jend = min(jc + chunk, L);
    const bool has_cur = pos0 < jend;                             // this chunk holds pos0
    const int R = kFusedR, hr = kFusedRope / 2;
    const int cu = tid & (kFusedNcu - 1), rs = tid / kFusedNcu;
    // small loads first (as mla_fused_kernel), then the weights, then the
    // chunk's first block of records
    const int ti = tid < hr ? tid : 0;
    const float* qr = a.q + (int64_t)a.H * a.nope + (int64_t)h * kFusedRope;
    const float qn = gld(a.q + (int64_t)h * a.nope + (tid < a.nope ? tid : 0));
    float x0 = gld(qr + ti), x1 = gld(qr + ti + hr);
    float k0 = gld(a.kva + kFusedDc + ti), k1 = gld(a.kva + kFusedDc + ti + hr);
    float rc = 1.f, rsn = 0.f;
    if (a.rc) { rc = gld(a.rc + (int64_t)pos0 * hr + ti); rsn = gld(a.rs + (int64_t)pos0 * hr + ti); }
    const float cx = gld(a.kva + (tid & (kFusedDc - 1))), cn = gld(a.k_norm + (tid & (kFusedDc - 1)));
    const float cx2 = gld(a.kva + (tid & 255) + 256);
    __builtin_amdgcn_sched_barrier(0);
    RawUnit wk[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int i = rs + kFusedRs * r;
        raw_issue<QT>(wk[r], a.wkvb, ((int64_t)h * a.nope + (i < a.nope ? i : 0)) * kFusedDc + 16 * cu);
    }
    __builtin_amdgcn_sched_barrier(0);
    float kv[kFusedPw][kFusedRec];
    fused_load_block(kv, a.cache, jc, wave, pos0, lane);
    __builtin_amdgcn_sched_barrier(0);
    if (tid < a.nope) s_qn[tid] = qn;
    if (tid < hr) {
        if (a.rc) {
            rope_pair(x0, x1, rc, rsn, x0, x1);
            rope_pair(k0, k1, rc, rsn, k0, k1);
        }
        s_q[kFusedDc + tid] = x0;
        s_q[kFusedDc + tid + hr] = x1;
        s_rec[kFusedDc + tid] = k0;
        s_rec[kFusedDc + tid + hr] = k1;
        if (h == 0 && has_cur) {
            float* rec = a.cache + (int64_t)pos0 * R;
            gst(rec + kFusedDc + tid, k0);
            gst(rec + kFusedDc + tid + hr, k1);
        }
    }
    if (tid < 256) {
        const float ss = wave_sum(fmaf(cx2, cx2, fmaf(cx, cx, 0.f)));
        if (lane == 0) s_red[wave] = ss;
    }
    __syncthreads();
    {
        float acc[16], bias = 0.f;
#pragma unroll
        for (int j = 0; j < 16; j++) acc[j] = 0.f;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int i = rs + kFusedRs * r;
            raw_fold<QT>(wk[r], i < a.nope ? s_qn[i] : 0.f, acc, bias);
        }
        f32x4* dst = (f32x4*)(s_part + rs * kFusedDc + 16 * cu);
#pragma unroll
        for (int q = 0; q < 4; q++)
            dst[q] = f32x4{acc[4 * q] - bias, acc[4 * q + 1] - bias, acc[4 * q + 2] - bias, acc[4 * q + 3] - bias};
    }
    if (tid < kFusedDc) {
        const float inv = 1.0f / sqrtf(((s_red[0] + s_red[1]) + (s_red[2] + s_red[3])) / (float)kFusedDc + a.eps);
        const float v = cx * inv * cn;
        s_rec[tid] = v;
        if (h == 0 && has_cur) gst(a.cache + (int64_t)pos0 * R + tid, v);
    }
    __syncthreads();
    if (tid < kFusedDc) {
        float t = 0.f;
#pragma unroll 8
        for (int r = 0; r < kFusedRs; r++) t += s_part[r * kFusedDc + tid];
        s_q[tid] = t;
    }
    __syncthreads();
    float qv[kFusedRec];
#pragma unroll
    for (int j = 0; j < kFusedRec; j++) qv[j] = s_q[lane + 64 * j];
    const float sc2 = a.scale * 1.44269504088896341f;
    float m = -INFINITY, l = 0.f, o[kFusedDc / 64];
#pragma unroll
    for (int j = 0; j < kFusedDc / 64; j++) o[j] = 0.f;
    for (int blk = jc; blk < jend; blk += kFusedBlock) {
        // the next block's records go out before this block is scored
        const bool more = blk + kFusedBlock < jend;           // uniform
        float kn[kFusedPw][kFusedRec];
        if (more) fused_load_block(kn, a.cache, blk + kFusedBlock, wave, pos0, lane);
        float sv[kFusedPw];
        float mb = -INFINITY;
#pragma unroll
        for (int i = 0; i < kFusedPw; i++) {
            const int p = blk + wave + 16 * i;
            sv[i] = -INFINITY;
            if (p < jend) {
                if (p == pos0) {
#pragma unroll
                    for (int j = 0; j < kFusedRec; j++) kv[i][j] = s_rec[lane + 64 * j];
                }
                float dot = 0.f;
#pragma unroll
                for (int j = 0; j < kFusedRec; j++) dot = fmaf(qv[j], kv[i][j], dot);
                sv[i] = wave_sum(dot) * sc2;
                mb = fmaxf(mb, sv[i]);
            }
        }
        if (mb != -INFINITY) {
            const float mn = fmaxf(m, mb), al = __builtin_amdgcn_exp2f(m - mn);
            l *= al;
#pragma unroll
            for (int j = 0; j < kFusedDc / 64; j++) o[j] *= al;
            m = mn;
#pragma unroll
            for (int i = 0; i < kFusedPw; i++) {
                if (sv[i] == -INFINITY) continue;
                const float pe = __builtin_amdgcn_exp2f(sv[i] - mn);
                l += pe;
#pragma unroll
                for (int j = 0; j < kFusedDc / 64; j++) o[j] = fmaf(pe, kv[i][j], o[j]);
            }
        }
        if (more) {
#pragma unroll
            for (int i = 0; i < kFusedPw; i++)
#pragma unroll
                for (int j = 0; j < kFusedRec; j++) kv[i][j] = kn[i][j];
        }
    }
#pragma unroll
    for (int j = 0; j < kFusedDc / 64; j++) s_part[wave * kFusedDc + lane + 64 * j] = o[j];
    if (lane == 0) { s_m[wave] = m; s_l[wave] = l; }
    __syncthreads();
    // merge of the 16 waves: the chunk's maximum, its sum and the
    // unnormalized latent partial, written for the combine kernel
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < 16; w++) M = fmaxf(M, s_m[w]);
    if (tid < kFusedDc) {
        float t = 0.f;
#pragma unroll
        for (int w = 0; w < 16; w++) {
            const float mw = s_m[w];
            t = fmaf(mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - M), s_part[w * kFusedDc + tid], t);
        }
        gst(a.ws_o + ((int64_t)c * a.H + h) * kFusedDc + tid, t);
    }
    if (tid == 0) {
        float den = 0.f;
#pragma unroll
        for (int w = 0; w < 16; w++) den = fmaf(s_m[w] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(s_m[w] - M), s_l[w], den);
        gst(a.ws_m + (int64_t)c * a.H + h, M);
        gst(a.ws_l + (int64_t)c * a.H + h, den);
    }
}

// grid (H, v/16), 256 threads: the chunk merge of head h,
// o_lat = sum_c 2^(M_c - M) partial_c / sum_c 2^(M_c - M) l_c over the
// chunks holding positions 0..pos0 (at most kChunkTarget), then 16 rows of
// out_h = W_vb_h o_lat, 4 per wave, 2 per half wave (a row's 32 units over
// the half's 32 lanes).  Thread = (float4 column tid & 127, chunk parity
// tid >> 7): 8 16-byte partial loads, the chunk maxima / sums and two W_vb
// units per thread, all issued at entry (one round trip).  Every workgroup
// of the head repeats the small merge.
template <int QT>
__global__ __launch_bounds__(256) void mla_combine_kernel(MlaArgs a) {
    __shared__ float s_w[kChunkTarget];
    __shared__ __align__(16) f32x4 s_half[kFusedDc / 4];
    __shared__ __align__(16) float s_lat[kFusedDc];
    __shared__ float s_red[8];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int pos0 = read_pos(a.start_pos, a.d_pos);
    if (pos0 < 0 || pos0 >= a.max_seq) return;
    const int nch = pos0 / chunk_of(a, pos0 + 1) + 1;       // <= kChunkTarget
    const int h = blockIdx.x;
    // this wave's 4 rows (v % 4 == 0; rows past v: a clamped row, not stored)
    const int i0 = 16 * blockIdx.y + 4 * wave;
    const bool rows_ok = i0 < a.v;
    const int64_t row0 = (int64_t)a.H * a.nope + (int64_t)h * a.v + (rows_ok ? i0 : 0);
    const int ul = lane & (kFusedNcu - 1), hw = lane >> 5;    // unit, half wave: rows i0 + 2 r + hw
    RawUnit wv[2];
#pragma unroll
    for (int r = 0; r < 2; r++) raw_issue<QT>(wv[r], a.wkvb, (row0 + 2 * r + hw) * kFusedDc + 16 * ul);
    const int t4 = tid & 127, cp = tid >> 7;
    f32x4 pv[kChunkTarget / 2];
#pragma unroll
    for (int i = 0; i < kChunkTarget / 2; i++) {
        const int cc = 2 * i + cp < nch ? 2 * i + cp : nch - 1;
        pv[i] = gld((const f32x4*)(a.ws_o + ((int64_t)cc * a.H + h) * kFusedDc) + t4);
    }
    const float mc = tid < nch ? gld(a.ws_m + (int64_t)tid * a.H + h) : -INFINITY;
    const float lc = tid < nch ? gld(a.ws_l + (int64_t)tid * a.H + h) : 0.f;
    const float mw = wave_max(mc);
    if (lane == 0) s_red[wave] = mw;
    __syncthreads();
    const float M = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
    const float w = tid < nch ? __builtin_amdgcn_exp2f(mc - M) : 0.f;   // partial maxima in base-2 units
    if (tid < kChunkTarget) s_w[tid] = w;
    const float lw = wave_sum(w * lc);
    __syncthreads();
    if (lane == 0) s_red[4 + wave] = lw;
    // each parity's chunks (weight 0 past nch), then the two parities
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < kChunkTarget / 2; i++) acc += pv[i] * s_w[2 * i + cp];
    if (cp) s_half[t4] = acc;
    __syncthreads();
    const float inv_l = 1.0f / ((s_red[4] + s_red[5]) + (s_red[6] + s_red[7]));
    if (!cp) *(f32x4*)(s_lat + 4 * t4) = (acc + s_half[t4]) * inv_l;
    __syncthreads();
    float o2[2];
#pragma unroll
    for (int r = 0; r < 2; r++) {
        float pr = sum16(raw_dot<QT>(wv[r], s_lat + 16 * ul));
        pr += dpp_rows<0x142, 0xA>(pr);   // row_bcast:15: lane 31 = lanes 0..31, lane 63 = lanes 32..63
        o2[r] = pr;
    }
    if (rows_ok && (lane & 31) == 31) {
        gst(a.out + (int64_t)h * a.v + i0 + hw, o2[0]);
        gst(a.out + (int64_t)h * a.v + i0 + 2 + hw, o2[1]);
    }
}

// ---------------------------------------------------------------------------
// A prompt from position 0 in the expanded form of the reference's prefill
// (deepseek_mla_layer.cu:180-217: one causal attention over all prompt rows
// with K = [W_kb c | RoPE(k_pe)] and V = W_vb c per head):
//   mla_rows_kernel:   each row's latent record into the cache (the same
//                      operations as the decode kernels' append), its
//                      normalized c into a contiguous matrix and its query
//                      [q_nope | RoPE(q_rope)] per head;
//   one T-row product of the two halves of w_kv_b (K_nope, V);
//   mla_expand_kernel: per row and head, K = [K_nope | RoPE(k_pe)] and V
//                      padded with zeros to the key width;
//   causal attention over the T rows (rina_hip_gqa_attention with H KV
//   heads of width nope + rope: scale 1/sqrt(nope + rope)), then the value
//   columns of each head's output.
// ---------------------------------------------------------------------------

// grid T, 256 threads: row t at position start_pos + t (dc <= 512, rope / 2 <= 256)
__global__ __launch_bounds__(256) void mla_rows_kernel(MlaArgs a, float* c_rows, float* q_full) {
    __shared__ float s_red[4];
    const int tid = threadIdx.x, t = blockIdx.x;
    const int pos = a.start_pos + (int)t;
    const int R = a.dc + a.rope, hr = a.rope / 2, D = a.nope + a.rope;
    const float* kva = a.kva + (int64_t)t * R;
    const int k0 = tid < a.dc ? tid : 0, k1 = tid + 256 < a.dc ? tid + 256 : 0, jr = tid < hr ? tid : 0;
    const float x0 = gld(kva + k0), x1 = gld(kva + k1);
    const float n0 = gld(a.k_norm + k0), n1 = gld(a.k_norm + k1);
    float p0 = gld(kva + a.dc + jr), p1 = gld(kva + a.dc + (hr ? jr + hr : 0));
    const float* tc = a.rc ? a.rc : kva;
    const float* ts = a.rs ? a.rs : kva;
    const float cc = gld(tc + (a.rc ? (int64_t)pos * hr + jr : 0)), sn = gld(ts + (a.rs ? (int64_t)pos * hr + jr : 0));
    float ss = (tid < a.dc ? x0 * x0 : 0.f);
    ss = fmaf(tid + 256 < a.dc ? x1 : 0.f, tid + 256 < a.dc ? x1 : 0.f, ss);
    ss = wave_sum(ss);
    if ((tid & 63) == 0) s_red[tid >> 6] = ss;
    // the query rows of every head: q_nope as it is, q_rope rotated at pos
    const float* q = a.q + (int64_t)t * a.H * D;
    float* qo = q_full + (int64_t)t * a.H * D;
    for (int i = tid; i < a.H * D; i += 256) {
        const int h = i / D, e = i % D;
        float v;
        if (e < a.nope) {
            v = gld(q + (int64_t)h * a.nope + e);
        } else {
            const int j = e - a.nope, jj = j < hr ? j : j - hr;
            const float* qr = q + (int64_t)a.H * a.nope + (int64_t)h * a.rope;
            float y0 = gld(qr + jj), y1 = gld(qr + jj + hr);
            if (a.rc) rope_pair(y0, y1, gld(a.rc + (int64_t)pos * hr + jj), gld(a.rs + (int64_t)pos * hr + jj), y0, y1);
            v = j < hr ? y0 : y1;
        }
        gst(qo + i, v);
    }
    __syncthreads();
    const float inv = 1.0f / sqrtf(((s_red[0] + s_red[1]) + (s_red[2] + s_red[3])) / (float)a.dc + a.eps);
    float* rec = a.cache + (int64_t)pos * R;
    float* cr = c_rows + (int64_t)t * a.dc;
    if (tid < a.dc) { const float v = x0 * inv * n0; gst(rec + tid, v); gst(cr + tid, v); }
    if (tid + 256 < a.dc) { const float v = x1 * inv * n1; gst(rec + tid + 256, v); gst(cr + tid + 256, v); }
    if (tid < hr) {
        if (a.rc) rope_pair(p0, p1, cc, sn, p0, p1);
        gst(rec + a.dc + tid, p0);
        gst(rec + a.dc + tid + hr, p1);
    }
}

// grid (T, H), 256 threads (nope + rope <= 256): K and V rows of head h at row t
__global__ __launch_bounds__(256) void mla_expand_kernel(MlaArgs a, const float* k_nope, const float* v_rows,
                                                         float* k_full, float* v_full) {
    const int tid = threadIdx.x, t = blockIdx.x, h = blockIdx.y;
    const int D = a.nope + a.rope;
    if (tid >= D) return;
    const int64_t o = ((int64_t)t * a.H + h) * D + tid;
    const float kv = tid < a.nope ? gld(k_nope + ((int64_t)t * a.H + h) * a.nope + tid)
                                  : gld(a.cache + (int64_t)(a.start_pos + t) * (a.dc + a.rope) + a.dc + (tid - a.nope));
    gst(k_full + o, kv);
    gst(v_full + o, tid < a.v ? gld(v_rows + ((int64_t)t * a.H + h) * a.v + tid) : 0.f);
}

// ---------------------------------------------------------------------------
// MoE
// ---------------------------------------------------------------------------

// deepseek_mla_layer.cu:310-326: softmax over E logits (serial fp32 sum of
// the exponentials in expert order), then the top-k of the reference's
// insertion loop.  That loop keeps the k largest probabilities with strict
// ">" (of equal values the earlier expert stays) in ascending order, equal
// values ending up later-expert first.  Here every expert computes its rank
// against the others in parallel, which gives the same set and order.
// grid = rows: workgroup r selects from logits row r into ids / probs row r
__global__ __launch_bounds__(256) void moe_topk_kernel(const float* lg, int E, int k, int* ids, float* probs) {
    __shared__ float s_p[256];
    __shared__ float s_red[4];
    __shared__ float s_inv;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    lg += (int64_t)blockIdx.x * E;
    ids += (int64_t)blockIdx.x * k;
    probs += (int64_t)blockIdx.x * k;
    const float x = tid < E ? gld(lg + tid) : -INFINITY;
    const float wm = wave_max(x);
    if (lane == 0) s_red[wave] = wm;
    __syncthreads();
    const float mx = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
    const float ex = tid < E ? expf(x - mx) : 0.f;
    s_p[tid] = ex;
    __syncthreads();
    if (tid == 0) {
        float sum = 0.f;
        for (int e = 0; e < E; e++) sum += s_p[e];
        s_inv = 1.0f / sum;
    }
    __syncthreads();
    const float p = ex * s_inv;
    __syncthreads();
    s_p[tid] = p;
    __syncthreads();
    if (tid < E) {
        int above = 0;
        for (int e = 0; e < E; e++) {
            const float q = s_p[e];
            above += (q > p) || (q == p && e < tid);
        }
        if (above < k) {
            gst(ids + (k - 1 - above), tid);
            gst(probs + (k - 1 - above), p);
        }
    }
}

// prompt rows of the MoE block, grouped by expert: X[i] = a2[idx[i]]
__global__ __launch_bounds__(256) void moe_gather_kernel(const float* a2, const int* idx, int d, float* X) {
    const float* src = a2 + (int64_t)gld(idx + blockIdx.x) * d;
    float* dst = X + (int64_t)blockIdx.x * d;
    for (int c = threadIdx.x; c < d; c += 256) gst(dst + c, gld(src + c));
}

// h[idx[i]] += pr[i] * Y[i]: one expert's rows (distinct rows within a launch)
__global__ __launch_bounds__(256) void moe_scatter_kernel(float* h, const int* idx, const float* pr, const float* Y,
                                                          int d) {
    float* dst = h + (int64_t)gld(idx + blockIdx.x) * d;
    const float* src = Y + (int64_t)blockIdx.x * d;
    const float p = gld(pr + blockIdx.x);
    for (int c = threadIdx.x; c < d; c += 256) gst(dst + c, fmaf(p, gld(src + c), gld(dst + c)));
}

struct MoeArgs {
    const float* x;        // [d] (post-norm activation)
    const uint8_t* wg;     // gate experts [E] x [ffn, d]
    const uint8_t* wu;     // up experts
    const uint8_t* wd;     // down experts [E] x [d, ffn]
    int qt;
    int64_t stride_gu, stride_dn;
    const int* ids;        // [k] ascending by probability, -1 = none
    const float* probs;    // [k]
    int k, d, ffn, E;
    float* G;              // [k][ffn] SiLU(gate) * up
    const float* shared;   // [d] shared-expert output
    float* h;              // [d] residual stream: h += shared + sum_k p_k y_k
};

// one wave per (slot, row) of the selected experts' gate/up
__global__ __launch_bounds__(256) void moe_gate_up_kernel(MoeArgs a) {
    extern __shared__ __align__(16) float s_x[];
    __shared__ int s_ids[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    stage_lds(s_x, a.x, a.d);
    if (tid < a.k) s_ids[tid] = gld(a.ids + tid);
    __syncthreads();
    const int rows = a.k * a.ffn;                 // even: ffn % 16 == 0
    for (int r = 2 * (blockIdx.x * 4 + wave); r < rows; r += 2 * gridDim.x * 4) {
        int e2[2];
        int64_t i2[2];
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const int e = s_ids[(r + t) / a.ffn];
            e2[t] = (e >= 0 && e < a.E) ? e : -1;
            i2[t] = (r + t) % a.ffn;
        }
        const uint8_t* const w4[4] = {a.wg + (int64_t)max(e2[0], 0) * a.stride_gu, a.wu + (int64_t)max(e2[0], 0) * a.stride_gu,
                                      a.wg + (int64_t)max(e2[1], 0) * a.stride_gu, a.wu + (int64_t)max(e2[1], 0) * a.stride_gu};
        const int64_t r4[4] = {i2[0], i2[0], i2[1], i2[1]};
        const float* const x4[4] = {s_x, s_x, s_x, s_x};
        float o4[4];
        rows_dot<4>(w4, a.qt, r4, a.d, x4, lane, o4);
        if (lane < 2) {
            const float g = lane == 0 ? o4[0] : o4[2], u = lane == 0 ? o4[1] : o4[3];
            gst(a.G + r + lane, e2[lane] >= 0 ? (g / (1.0f + expf(-g))) * u : 0.f);
        }
    }
}

// one wave per output row i: acc = shared[i]; acc += p_j y_j (ascending j); h[i] += acc
__global__ __launch_bounds__(256) void moe_down_kernel(MoeArgs a) {
    extern __shared__ __align__(16) float s_g[];
    __shared__ int s_ids[16];
    __shared__ float s_p[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    stage_lds(s_g, a.G, a.k * a.ffn);
    if (tid < a.k) { s_ids[tid] = gld(a.ids + tid); s_p[tid] = gld(a.probs + tid); }
    __syncthreads();
    for (int i = blockIdx.x * 4 + wave; i < a.d; i += gridDim.x * 4) {
        float acc = gld(a.shared + i);
        for (int j0 = 0; j0 < a.k; j0 += 6) {
            const uint8_t* w4[6];
            int64_t r4[6];
            const float* x4[6];
#pragma unroll
            for (int t = 0; t < 6; t++) {
                const int j = min(j0 + t, a.k - 1);
                const int e = s_ids[j];
                w4[t] = a.wd + (int64_t)((e >= 0 && e < a.E) ? e : 0) * a.stride_dn;
                r4[t] = i;
                x4[t] = s_g + j * a.ffn;
            }
            float y4[6];
            rows_dot<6>(w4, a.qt, r4, a.ffn, x4, lane, y4);
#pragma unroll
            for (int t = 0; t < 6; t++) {
                const int j = j0 + t;
                if (j < a.k) {
                    const int e = s_ids[j];
                    if (e >= 0 && e < a.E) acc = fmaf(s_p[j], y4[t], acc);   // ascending j, as the saxpy chain
                }
            }
        }
        if (lane == 0) gst(a.h + i, gld(a.h + i) + acc);
    }
}

bool unit_qt(int qt) {
    return qt == RINA_QT_GGML_Q2_K || qt == RINA_QT_Q4_0 || qt == RINA_QT_Q4_0F || qt == RINA_QT_FP32;
}

// positions per split workgroup: a multiple of kMlaChunk that keeps the
// chunk count at most kMlaMaxChunks (the out kernel merges them at once)
int mla_chunk_len(int max_pos) {
    const int blocks = (max_pos + kMlaChunk - 1) / kMlaChunk;
    return kMlaChunk * ((blocks + kMlaMaxChunks - 1) / kMlaMaxChunks);
}
int mla_nchunk(int max_pos) {
    const int cl = mla_chunk_len(max_pos);
    return (max_pos + cl - 1) / cl;
}
// chunk partials the workspace holds: the most the split kernel
// (mla_nchunk) or the chunk kernel (at most kChunkTarget chunks of whole
// 64-position blocks) uses for up to max_pos positions
int mla_ws_chunks(int max_pos) {
    return std::min(kMlaMaxChunks, (max_pos + kMlaChunk - 1) / kMlaChunk);
}

// shapes mla_fused_kernel is built for (the DeepSeek-V2 latent width)
bool mla_fused_ok(int qt, int nope, int rope, int v, int dc) {
    return (qt == RINA_QT_GGML_Q2_K || qt == RINA_QT_Q4_0F || qt == RINA_QT_Q4_0) && dc == kFusedDc &&
           rope == kFusedRope && nope <= 128 && v <= 128;
}

}  // namespace

extern "C" size_t rina_hip_mla_attention_workspace(int H, int dc, int rope, int max_pos) {
    if (H < 1 || dc < 1 || max_pos < 1) return 0;
    // the most chunks any call with up to max_pos positions uses (a shorter
    // cache can take more, shorter chunks)
    const size_t nch = (size_t)mla_ws_chunks(max_pos);
    return ((size_t)H * (dc + rope) + nch * H * (2 + (size_t)dc)) * sizeof(float);
}

extern "C" size_t rina_hip_mla_cache_bytes(int dc, int rope, int max_seq) {
    return (size_t)max_seq * (dc + rope) * sizeof(float);
}

extern "C" int rina_hip_mla_decode_attention_ex(const float* q, const float* kva, const float* k_norm, float eps,
                                                const float* rope_cos, const float* rope_sin, const void* w_kv_b,
                                                int qt_kv_b, float* cache, int H, int nope, int rope, int v_dim,
                                                int dc, int start_pos, const int* d_pos, int max_seq, int pos_hint,
                                                float* out, void* workspace, size_t ws_bytes, void* stream) {
    if (!q || !kva || !k_norm || !w_kv_b || !cache || !out || H < 1 || nope < 1 || v_dim < 1 || max_seq < 1)
        return RINA_ERR_ARG;
    if (!unit_qt(qt_kv_b)) return RINA_ERR_QTYPE;
    if ((!rope_cos) != (!rope_sin)) return RINA_ERR_ARG;
    if (dc % 64 || dc > 512 || rope % 2 || rope < 0 || dc + rope > 64 * kMaxRecLanes || v_dim % 4 ||
        (256 % (dc / 64)) || nope > kPrepRows * (256 / (dc / 64)) || max_seq > 32768)
        return RINA_ERR_SHAPE;
    if (!d_pos && (start_pos < 0 || start_pos >= max_seq)) return RINA_ERR_RANGE;
    if (((uintptr_t)w_kv_b | (uintptr_t)q | (uintptr_t)cache) % 16 || (uintptr_t)w_kv_b % 4) return RINA_ERR_SHAPE;
    const int max_pos = d_pos ? max_seq : start_pos + 1;
    const size_t need = rina_hip_mla_attention_workspace(H, dc, rope, max_pos);
    if (!workspace || ws_bytes < need) return RINA_ERR_WORKSPACE;
    MlaArgs a{};
    a.q = q; a.kva = kva; a.k_norm = k_norm; a.eps = eps; a.rc = rope_cos; a.rs = rope_sin;
    a.wkvb = (const uint8_t*)w_kv_b; a.qt = qt_kv_b; a.cache = cache; a.out = out;
    a.H = H; a.nope = nope; a.rope = rope; a.v = v_dim; a.dc = dc;
    a.start_pos = start_pos; a.max_seq = max_seq; a.d_pos = d_pos; a.chunk = mla_chunk_len(max_pos);
    a.scale = 1.0f / sqrtf((float)(nope + rope));
    const int nch = mla_ws_chunks(max_pos);
    a.ws_q = (float*)workspace;
    a.ws_m = a.ws_q + (size_t)H * (dc + rope);
    a.ws_l = a.ws_m + (size_t)nch * H;
    a.ws_o = a.ws_l + (size_t)nch * H;
    hipStream_t st = as_stream(stream);
    // positions the launch will see: known without d_pos, else the caller's
    // bound (any position is computed correctly by either path)
    const int lmax = d_pos ? (pos_hint >= 0 ? std::min(pos_hint + 1, max_seq) : max_seq) : start_pos + 1;
    if (lmax <= kFusedMaxPos && mla_fused_ok(qt_kv_b, nope, rope, v_dim, dc)) {
        const dim3 grid(H, kFusedY);
        if (qt_kv_b == RINA_QT_GGML_Q2_K) hipLaunchKernelGGL(mla_fused_kernel<RINA_QT_GGML_Q2_K>, grid, dim3(1024), 0, st, a);
        else if (qt_kv_b == RINA_QT_Q4_0F) hipLaunchKernelGGL(mla_fused_kernel<RINA_QT_Q4_0F>, grid, dim3(1024), 0, st, a);
        else hipLaunchKernelGGL(mla_fused_kernel<RINA_QT_Q4_0>, grid, dim3(1024), 0, st, a);
        RINA_LAUNCH_CHECK();
        return RINA_OK;
    }
    if (mla_fused_ok(qt_kv_b, nope, rope, v_dim, dc)) {
        // about kChunkTarget chunks of whole 64-position blocks (fewer
        // while the positions are few): every chunk workgroup repeats
        // q_lat and W_vb, so fewer, longer chunks win once a workgroup per
        // CU is reached
        a.chunk = kFusedBlock;
        a.nslot = std::min(kChunkTarget, (max_pos + kFusedBlock - 1) / kFusedBlock);
        const int ncc = a.nslot;
        const dim3 grid((ncc + 7) / 8 * 8, H);
        if (qt_kv_b == RINA_QT_GGML_Q2_K) hipLaunchKernelGGL(mla_chunk_kernel<RINA_QT_GGML_Q2_K>, grid, dim3(1024), 0, st, a);
        else if (qt_kv_b == RINA_QT_Q4_0F) hipLaunchKernelGGL(mla_chunk_kernel<RINA_QT_Q4_0F>, grid, dim3(1024), 0, st, a);
        else hipLaunchKernelGGL(mla_chunk_kernel<RINA_QT_Q4_0>, grid, dim3(1024), 0, st, a);
        RINA_LAUNCH_CHECK();
        const dim3 cgrid(H, (v_dim + 15) / 16);
        if (qt_kv_b == RINA_QT_GGML_Q2_K) hipLaunchKernelGGL(mla_combine_kernel<RINA_QT_GGML_Q2_K>, cgrid, dim3(256), 0, st, a);
        else if (qt_kv_b == RINA_QT_Q4_0F) hipLaunchKernelGGL(mla_combine_kernel<RINA_QT_Q4_0F>, cgrid, dim3(256), 0, st, a);
        else hipLaunchKernelGGL(mla_combine_kernel<RINA_QT_Q4_0>, cgrid, dim3(256), 0, st, a);
        RINA_LAUNCH_CHECK();
        return RINA_OK;
    }
    hipLaunchKernelGGL(mla_prep_kernel, dim3(H + 1, 4), dim3(256), 0, st, a);
    RINA_LAUNCH_CHECK();
    // chunks padded to the 8 XCDs: every head of a chunk reads the same
    // latent records, fetched into one L2 (padding workgroups start past
    // max_seq and return)
    const int nsp = mla_nchunk(max_pos);
    hipLaunchKernelGGL(mla_split_kernel, dim3((nsp + 7) / 8 * 8, H), dim3(64 * kSplitWaves), 0, st, a);
    RINA_LAUNCH_CHECK();
    hipLaunchKernelGGL(mla_out_kernel, dim3(H, (v_dim + 15) / 16), dim3(256), 0, st, a);
    RINA_LAUNCH_CHECK();
    return RINA_OK;
}

extern "C" int rina_hip_mla_fused_positions(void) { return kFusedMaxPos; }

extern "C" int rina_hip_mla_decode_attention(const float* q, const float* kva, const float* k_norm, float eps,
                                             const float* rope_cos, const float* rope_sin, const void* w_kv_b,
                                             int qt_kv_b, float* cache, int H, int nope, int rope, int v_dim, int dc,
                                             int start_pos, const int* d_pos, int max_seq, float* out,
                                             void* workspace, size_t ws_bytes, void* stream) {
    return rina_hip_mla_decode_attention_ex(q, kva, k_norm, eps, rope_cos, rope_sin, w_kv_b, qt_kv_b, cache, H, nope,
                                            rope, v_dim, dc, start_pos, d_pos, max_seq, -1, out, workspace, ws_bytes,
                                            stream);
}

extern "C" size_t rina_hip_mla_prompt_workspace(int T, int H, int nope, int rope, int v_dim, int dc) {
    if (T < 1 || H < 1 || nope < 1 || v_dim < 1 || dc < 1 || rope < 0) return 0;
    const size_t D = (size_t)nope + rope, t = (size_t)T;
    // c rows | K_nope | V | K, V, Q, O at width nope + rope (16-byte aligned parts)
    auto up4 = [](size_t n) { return (n + 3) / 4 * 4; };
    return sizeof(float) * (up4(t * dc) + up4(t * H * nope) + up4(t * H * v_dim) + 4 * up4(t * H * D));
}

extern "C" int rina_hip_mla_prompt_attention(const float* q, const float* kva, const float* k_norm, float eps,
                                             const float* rope_cos, const float* rope_sin, const void* w_kv_b,
                                             int qt_kv_b, float* cache, int H, int nope, int rope, int v_dim, int dc,
                                             int T, int max_seq, float* out, void* workspace, size_t ws_bytes,
                                             void* stream) {
    if (!q || !kva || !k_norm || !w_kv_b || !cache || !out || H < 1 || nope < 1 || v_dim < 1 || dc < 1 || T < 1 ||
        max_seq < 1 || rope < 0 || rope % 2)
        return RINA_ERR_ARG;
    if (T > max_seq) return RINA_ERR_RANGE;
    if (dc > 512 || rope / 2 > 256 || nope + rope > 256 || v_dim > nope + rope) return RINA_ERR_SHAPE;
    int64_t vb_off;   // byte offset of the W_vb rows (after the H*nope W_kb rows)
    const int64_t nkb = (int64_t)H * nope * dc;
    if (qt_kv_b == RINA_QT_GGML_Q2_K) { if (nkb % 256) return RINA_ERR_SHAPE; vb_off = nkb / 256 * 84; }
    else if (qt_kv_b == RINA_QT_Q4_0) { if (nkb % 32) return RINA_ERR_SHAPE; vb_off = nkb / 32 * 18; }
    else if (qt_kv_b == RINA_QT_Q4_0F) { if (nkb % 32) return RINA_ERR_SHAPE; vb_off = nkb / 32 * 20; }
    else if (qt_kv_b == RINA_QT_FP32) vb_off = nkb * 4;
    else return RINA_ERR_QTYPE;
    const size_t need = rina_hip_mla_prompt_workspace(T, H, nope, rope, v_dim, dc);
    if (!workspace || ws_bytes < need || (uintptr_t)workspace % 16) return RINA_ERR_WORKSPACE;
    const int D = nope + rope;
    auto up4 = [](size_t n) { return (n + 3) / 4 * 4; };
    float* c_rows = (float*)workspace;
    float* k_nope = c_rows + up4((size_t)T * dc);
    float* v_rows = k_nope + up4((size_t)T * H * nope);
    float* k_full = v_rows + up4((size_t)T * H * v_dim);
    float* v_full = k_full + up4((size_t)T * H * D);
    float* q_full = v_full + up4((size_t)T * H * D);
    float* o_full = q_full + up4((size_t)T * H * D);
    MlaArgs a{};
    a.q = q; a.kva = kva; a.k_norm = k_norm; a.eps = eps; a.rc = rope_cos; a.rs = rope_sin;
    a.wkvb = (const uint8_t*)w_kv_b; a.qt = qt_kv_b; a.cache = cache; a.out = out;
    a.H = H; a.nope = nope; a.rope = rope; a.v = v_dim; a.dc = dc; a.start_pos = 0; a.max_seq = max_seq;
    hipStream_t st = as_stream(stream);
    hipLaunchKernelGGL(mla_rows_kernel, dim3(T), dim3(256), 0, st, a, c_rows, q_full);
    RINA_LAUNCH_CHECK();
    rina_linear_seg segs[2] = {{w_kv_b, nullptr, k_nope, H * nope},
                               {(const uint8_t*)w_kv_b + vb_off, nullptr, v_rows, H * v_dim}};
    int rc = rina_hip_linear_fused(segs, 2, qt_kv_b, c_rows, T, dc, RINA_EPI_STORE, RINA_PRO_NONE, nullptr, 0.f, stream);
    if (rc) return rc;
    hipLaunchKernelGGL(mla_expand_kernel, dim3(T, H), dim3(256), 0, st, a, k_nope, v_rows, k_full, v_full);
    RINA_LAUNCH_CHECK();
    rc = rina_hip_gqa_attention(q_full, k_full, v_full, k_full, v_full, RINA_KV_FP32, 0, nullptr, nullptr, T, H, H, D,
                                0, nullptr, max_seq, o_full, nullptr, 0, stream);
    if (rc) return rc;
    // the value columns of every (row, head)
    if (hipMemcpy2DAsync(out, sizeof(float) * v_dim, o_full, sizeof(float) * D, sizeof(float) * v_dim, (size_t)T * H,
                         hipMemcpyDeviceToDevice, st) != hipSuccess)
        return RINA_ERR_HIP;
    return RINA_OK;
}

extern "C" int rina_hip_moe_topk(const float* logits, int n_experts, int k, int* ids, float* probs, void* stream) {
    if (!logits || !ids || !probs || n_experts < 1 || n_experts > 256 || k < 1 || k > 16 || k > n_experts)
        return RINA_ERR_ARG;
    hipLaunchKernelGGL(moe_topk_kernel, dim3(1), dim3(256), 0, as_stream(stream), logits, n_experts, k, ids, probs);
    RINA_LAUNCH_CHECK();
    return RINA_OK;
}

extern "C" size_t rina_hip_moe_workspace(int k, int ffn) { return (size_t)k * ffn * sizeof(float); }

// ---------------------------------------------------------------------------
// The MoE block over a prompt's T rows (forward_moe, deepseek_mla_layer.cu:
// 291-350, for every row at once): the rows' ln2 norm and fp32 router
// logits as T-row products, the top-k of every row, the shared experts as
// T-row products added to h, then one expert at a time (ascending id) its
// selected rows gathered, its gate/up (SiLU * up) and down products over
// them, and h[row] += p * y.  The selection comes to the host once to group
// the rows (the stream is synchronized there).
// ---------------------------------------------------------------------------
namespace {
size_t up4f(size_t n) { return (n + 3) / 4 * 4; }
}

extern "C" size_t rina_hip_moe_rows_workspace(int T, int d, int E, int k, int F, int S) {
    if (T < 1 || d < 1 || E < 1 || k < 1 || F < 1 || S < 0) return 0;
    const size_t t = (size_t)T, tk = t * k;
    // a2 | logits | probs | ids | G_shared | X | G | Y | idx | pr
    return sizeof(float) * (up4f(t * d) + up4f(t * E) + 2 * up4f(tk) + up4f(t * S) + up4f(tk * d) + up4f(tk * F) +
                            up4f(tk * d) + 2 * up4f(tk));
}

extern "C" int rina_hip_moe_rows(float* h, int T, const float* ln2, float eps, const void* gate_inp, int qt_inp,
                                 const void* gate_sh, const void* up_sh, const void* down_sh, int S, int qt_sh,
                                 const void* gate_exps, const void* up_exps, const void* down_exps, int qt_exps,
                                 int64_t stride_gu, int64_t stride_dn, int E, int k, int d, int F, void* workspace,
                                 size_t ws_bytes, void* stream) {
    if (!h || !ln2 || !gate_inp || !gate_exps || !up_exps || !down_exps || T < 1 || E < 1 || E > 256 || k < 1 ||
        k > 16 || k > E || d < 1 || F < 1 || S < 0 || (S > 0 && (!gate_sh || !up_sh || !down_sh)))
        return RINA_ERR_ARG;
    const size_t need = rina_hip_moe_rows_workspace(T, d, E, k, F, S);
    if (!workspace || ws_bytes < need || (uintptr_t)workspace % 16) return RINA_ERR_WORKSPACE;
    hipStream_t st = as_stream(stream);
    const size_t t = (size_t)T, tk = t * k;
    float* a2 = (float*)workspace;
    float* logits = a2 + up4f(t * d);
    float* probs = logits + up4f(t * E);
    int* ids = (int*)(probs + up4f(tk));
    float* gsh = (float*)ids + up4f(tk);
    float* X = gsh + up4f(t * S);
    float* G = X + up4f(tk * d);
    float* Y = G + up4f(tk * F);
    int* idx = (int*)(Y + up4f(tk * d));
    float* pr = (float*)idx + up4f(tk);
    int rc;
    if ((rc = rina_hip_rms_norm(h, a2, ln2, T, d, eps, stream))) return rc;
    rina_linear_seg sr{gate_inp, nullptr, logits, E};
    if ((rc = rina_hip_linear_fused(&sr, 1, qt_inp, a2, T, d, RINA_EPI_STORE, RINA_PRO_NONE, nullptr, 0.f, stream)))
        return rc;
    hipLaunchKernelGGL(moe_topk_kernel, dim3(T), dim3(256), 0, st, logits, E, k, ids, probs);
    RINA_LAUNCH_CHECK();
    if (S > 0) {
        rina_linear_seg su{gate_sh, up_sh, gsh, S};
        if ((rc = rina_hip_linear_fused(&su, 1, qt_sh, a2, T, d, RINA_EPI_SWIGLU, RINA_PRO_NONE, nullptr, 0.f, stream)))
            return rc;
        rina_linear_seg sd{down_sh, nullptr, h, d};
        if ((rc = rina_hip_linear_fused(&sd, 1, qt_sh, gsh, T, S, RINA_EPI_ADD, RINA_PRO_NONE, nullptr, 0.f, stream)))
            return rc;
    }
    // the selection on the host: rows grouped by expert, ascending
    std::vector<int> hid(tk);
    std::vector<float> hpr(tk);
    if (hipMemcpyAsync(hid.data(), ids, tk * sizeof(int), hipMemcpyDeviceToHost, st) != hipSuccess ||
        hipMemcpyAsync(hpr.data(), probs, tk * sizeof(float), hipMemcpyDeviceToHost, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess)
        return RINA_ERR_HIP;
    std::vector<int> cnt(E + 1, 0), gi(tk), off(E + 1, 0);
    std::vector<float> gp(tk);
    for (size_t i = 0; i < tk; i++)
        if (hid[i] >= 0 && hid[i] < E) cnt[hid[i]]++;
    for (int e = 0; e < E; e++) off[e + 1] = off[e] + cnt[e];
    std::vector<int> fill(off.begin(), off.end() - 1);
    for (size_t i = 0; i < tk; i++) {
        const int e = hid[i];
        if (e < 0 || e >= E) continue;
        gi[fill[e]] = (int)(i / k);
        gp[fill[e]++] = hpr[i];
    }
    const int n_sel = off[E];
    if (n_sel > 0 &&
        (hipMemcpyAsync(idx, gi.data(), sizeof(int) * n_sel, hipMemcpyHostToDevice, st) != hipSuccess ||
         hipMemcpyAsync(pr, gp.data(), sizeof(float) * n_sel, hipMemcpyHostToDevice, st) != hipSuccess)) {
        (void)hipStreamSynchronize(st);
        return RINA_ERR_HIP;
    }
    for (int e = 0; e < E && rc == RINA_OK; e++) {
        const int n = cnt[e];
        if (!n) continue;
        const int o = off[e];
        float* Xe = X + (size_t)o * d;
        float* Ge = G + (size_t)o * F;
        float* Ye = Y + (size_t)o * d;
        hipLaunchKernelGGL(moe_gather_kernel, dim3(n), dim3(256), 0, st, a2, idx + o, d, Xe);
        if (hipGetLastError() != hipSuccess) { rc = RINA_ERR_HIP; break; }
        rina_linear_seg sg{(const uint8_t*)gate_exps + e * stride_gu, (const uint8_t*)up_exps + e * stride_gu, Ge, F};
        if ((rc = rina_hip_linear_fused(&sg, 1, qt_exps, Xe, n, d, RINA_EPI_SWIGLU, RINA_PRO_NONE, nullptr, 0.f, stream)))
            break;
        rina_linear_seg sd{(const uint8_t*)down_exps + e * stride_dn, nullptr, Ye, d};
        if ((rc = rina_hip_linear_fused(&sd, 1, qt_exps, Ge, n, F, RINA_EPI_STORE, RINA_PRO_NONE, nullptr, 0.f, stream)))
            break;
        hipLaunchKernelGGL(moe_scatter_kernel, dim3(n), dim3(256), 0, st, h, idx + o, pr + o, Ye, d);
        if (hipGetLastError() != hipSuccess) rc = RINA_ERR_HIP;
    }
    // the host lists are sources of queued copies: wait before they go
    if (hipStreamSynchronize(st) != hipSuccess && rc == RINA_OK) rc = RINA_ERR_HIP;
    return rc;
}

extern "C" int rina_hip_moe_ffn(const float* x, const void* gate_exps, const void* up_exps, const void* down_exps,
                                int qt, int64_t stride_gu, int64_t stride_dn, int n_experts, const int* ids,
                                const float* probs, int k, int d, int ffn, const float* shared_out, float* h,
                                void* workspace, size_t ws_bytes, void* stream) {
    if (!x || !gate_exps || !up_exps || !down_exps || !ids || !probs || !shared_out || !h || k < 1 || d < 1 ||
        ffn < 1 || n_experts < 1)
        return RINA_ERR_ARG;
    if (!unit_qt(qt)) return RINA_ERR_QTYPE;
    if (d % 16 || ffn % 16 || k > 16 || (size_t)k * ffn * 4 > 64 * 1024 || (size_t)d * 4 > 64 * 1024)
        return RINA_ERR_SHAPE;
    if (!workspace || ws_bytes < rina_hip_moe_workspace(k, ffn)) return RINA_ERR_WORKSPACE;
    if (((uintptr_t)gate_exps | (uintptr_t)up_exps | (uintptr_t)down_exps) % 4 || stride_gu % 4 || stride_dn % 4)
        return RINA_ERR_SHAPE;
    MoeArgs a{};
    a.x = x; a.wg = (const uint8_t*)gate_exps; a.wu = (const uint8_t*)up_exps; a.wd = (const uint8_t*)down_exps;
    a.qt = qt; a.stride_gu = stride_gu; a.stride_dn = stride_dn; a.ids = ids; a.probs = probs;
    a.k = k; a.d = d; a.ffn = ffn; a.E = n_experts; a.G = (float*)workspace; a.shared = shared_out; a.h = h;
    hipStream_t st = as_stream(stream);
    const int cus = rina_num_cus();
    int g1 = (k * ffn / 2 + 3) / 4;
    if (g1 > cus * 4) g1 = cus * 4;
    hipLaunchKernelGGL(moe_gate_up_kernel, dim3(g1), dim3(256), (size_t)d * 4, st, a);
    RINA_LAUNCH_CHECK();
    int g2 = (d + 7) / 8;          // two rows per wave: the activations are staged once per 8 rows
    if (g2 > cus) g2 = cus;
    hipLaunchKernelGGL(moe_down_kernel, dim3(g2), dim3(256), (size_t)k * ffn * 4, st, a);
    RINA_LAUNCH_CHECK();
    return RINA_OK;
}
