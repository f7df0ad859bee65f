// Single-layer GQA attention over the (quantized) KV cache.
//
// Semantics (rina-engine/src/arch/gqa/gqa_layer.cu:192-270 with
// kernels/flash_fp32.cu:12-111 and build_qkv_fp32.cu:8-33): query row t sits
// at position pos0+t and attends causally to keys 0..pos0+t; keys/values
// below pos0 come from the cache (dequantized with the block rules of
// kernels/quantize.cu), the others from the current fp32 rows; query head h
// reads KV head h / (H/Hkv); score = (q.k) / sqrt(dh).
//
// Decode (T == 1, dh == 64): split-sequence.  A workgroup takes a chunk of
// positions and a group of HG KV heads whose records are contiguous
// in every cache layout (position-major, heads inside), so each position's
// bytes are consumed whole.  8 lanes cover one head's 64 dims (8 values per
// lane, dequantized in registers), the REP query heads of that KV head are
// reduced with DPP inside the 8-lane group.  Scores go to LDS, the chunk's
// softmax is formed there, V is accumulated in registers and the chunk
// writes (max, sum, O) partials; the last chunk to finish merges them.
#include "rina_common.hpp"
#include "kv_formats.hpp"

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kSub = 32;     // chunk granularity (a multiple of every sub-step)
constexpr int kMaxChunks = 64;  // chunk partials per head (chunk size adapts)

// Chunk length for a cache of max_pos positions: at most kMaxChunks
// partials per head, each a multiple of the kSub sub-step.
int chunk_len(int max_pos, int gran) {
    int per = (max_pos + kMaxChunks - 1) / kMaxChunks;
    per = (per + gran - 1) / gran * gran;
    return per < gran ? gran : per;
}

constexpr size_t kCounterBytes = 256;   // per-head-group completion counters

struct AttnArgs {
    const float* q;
    const float* kcur;
    const float* vcur;
    const uint8_t* ck;
    const uint8_t* cv;
    const float* rkc;
    const float* rks;
    float* out;
    float* ws_m;
    float* ws_l;
    float* ws_o;
    int mode, pre_rope, T, H, Hkv, dh, start_pos, max_seq, nchunk_max, chunk;
    const int* d_pos;
    int* counters;   // per head group, in the workspace; zero between calls
    void* ws;
    size_t ws_bytes;
    float scale;
};

// 8 consecutive values [v0, v0+8) of one position's record, v0 % 8 == 0.
template <int FMT>
__device__ __forceinline__ void load8(const uint8_t* base, int64_t v0, float (&o)[8]) {
    if (FMT == 0) {
        const f32x4* p = (const f32x4*)((const float*)base + v0);
        f32x4 a = gld(p), b = gld(p + 1);
        o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
        o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
        return;
    }
    constexpr int BB = kvq::block_bytes_c(FMT);
    const uint8_t* blk = base + (v0 >> 5) * BB;
    const int w = (int)(v0 & 31);
    float s = f16_to_f32(gld((const uint16_t*)blk));
    if (FMT == RINA_KVF_Q8_0) {
        const uint8_t* d = blk + 2 + w;
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
            uint32_t two = gld((const uint16_t*)(d + i));
            o[i] = (float)(int8_t)(two & 0xFF) * s;
            o[i + 1] = (float)(int8_t)(two >> 8) * s;
        }
    } else if (FMT == RINA_KVF_Q4_0) {
        uint32_t n = (uint32_t)gld((const uint16_t*)(blk + 2 + w / 2)) |
                     ((uint32_t)gld((const uint16_t*)(blk + 4 + w / 2)) << 16);
#pragma unroll
        for (int i = 0; i < 8; i++) o[i] = (float)((int)((n >> (4 * i)) & 0xF) - 7) * s;
    } else if (FMT == RINA_KVF_Q2_1) {
        uint32_t n = gld((const uint16_t*)(blk + 2 + w / 4));
#pragma unroll
        for (int i = 0; i < 8; i++) o[i] = (float)((int)((n >> (2 * i)) & 3) - 1) * s;
    } else {
        uint32_t bits = ((uint32_t)gld((const uint16_t*)(blk + 2)) | ((uint32_t)gld((const uint16_t*)(blk + 4)) << 16)) >> w;
#pragma unroll
        for (int i = 0; i < 8; i++) o[i] = ((bits >> i) & 1u) ? s : -s;
    }
}

// Chunk c of a head group covers positions [c*CS, c*CS+CS) in sub-steps of
// kSub positions; K and V of a sub-step are loaded together (one HBM round
// trip), scores are reduced in LDS and the chunk keeps an online softmax
// across sub-steps.  The last workgroup of a head group to finish (counter in
// the workspace, reset by that workgroup) merges the chunk partials, so no
// second launch and no memset node is needed.
template <int KF, int VF, int HG, int REP>
__global__ __launch_bounds__(256) void attn_decode_kernel(AttnArgs a) {
    constexpr int DH = 64;
    constexpr int LPP = 8 * HG;          // lanes per position record
    constexpr int PPW = 64 / LPP;        // positions per wave step
    constexpr int GS = 4 * PPW;          // positions per workgroup step
    constexpr int SUB = GS > 16 ? GS : 16;   // positions per sub-step (divides kSub)
    constexpr int NST = SUB / GS;            // steps per sub-step
    constexpr int QH = HG * REP;         // query heads in the group
    constexpr int KBB = kvq::block_bytes_c(KF), VBB = kvq::block_bytes_c(VF);
    static_assert(NST >= 1 && kSub % SUB == 0, "sub-step");
    __shared__ float s_lds[QH][SUB];
    __shared__ float s_alpha[QH];
    __shared__ float o_red[GS * QH * DH];
    __shared__ float s_hm[QH], s_hl[QH];
    __shared__ int s_last;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int pos0 = read_pos(a.start_pos, a.d_pos);
    if (pos0 < 0 || pos0 >= a.max_seq) return;     // capacity guard (host checks host-known positions)
    const int L = pos0 + 1;
    const int CS = a.chunk;
    const int c = blockIdx.x;
    const int j0 = c * CS;
    if (j0 >= L) return;
    const int ncv = min(CS, L - j0);
    const int kvd = a.Hkv * DH;
    const int hg0 = blockIdx.y * HG;
    const int64_t KREC = KF ? (int64_t)(kvd / 32) * KBB : (int64_t)kvd * 4;
    const int64_t VREC = VF ? (int64_t)(kvd / 32) * VBB : (int64_t)kvd * 4;

    const int slot = lane / LPP, lig = lane % LPP;
    const int kvl = lig >> 3;                       // kv head inside the group
    const int dim0 = (lig & 7) * 8;
    const int kvh = hg0 + kvl;
    const int64_t voff = (int64_t)kvh * DH + dim0;  // value offset inside a position record
    const int wslot = wave * PPW + slot;

    float qv[REP][8], ov[REP][8];
    float m_run = -INFINITY, l_run = 0.f;           // owned by threads tid < QH
    bool first = true;
    for (int sub = 0; sub < ncv; sub += SUB) {
        float kv[NST][8], vv[NST][8];
#pragma unroll
        for (int st = 0; st < NST; st++) {
            const int jl = sub + st * GS + wslot;
            const int j = j0 + jl;
#pragma unroll
            for (int i = 0; i < 8; i++) kv[st][i] = vv[st][i] = 0.f;
            if (jl < ncv) {
                if (j == pos0) {
                    load8<0>((const uint8_t*)a.kcur, voff, kv[st]);
                    load8<0>((const uint8_t*)a.vcur, voff, vv[st]);
                } else {
                    load8<KF>(a.ck + (int64_t)j * KREC, voff, kv[st]);
                    load8<VF>(a.cv + (int64_t)j * VREC, voff, vv[st]);
                }
            }
        }
        if (first) {
#pragma unroll
            for (int r = 0; r < REP; r++) {
                const f32x4* qp = (const f32x4*)(a.q + (int64_t)(kvh * REP + r) * DH + dim0);
                f32x4 x0 = gld(qp), x1 = gld(qp + 1);
                qv[r][0] = x0.x; qv[r][1] = x0.y; qv[r][2] = x0.z; qv[r][3] = x0.w;
                qv[r][4] = x1.x; qv[r][5] = x1.y; qv[r][6] = x1.z; qv[r][7] = x1.w;
#pragma unroll
                for (int i = 0; i < 8; i++) ov[r][i] = 0.f;
            }
            first = false;
        }
#pragma unroll
        for (int st = 0; st < NST; st++) {
            const int jl = sub + st * GS + wslot;
#pragma unroll
            for (int r = 0; r < REP; r++) {
                float p = 0.f;
#pragma unroll
                for (int i = 0; i < 8; i++) p = fmaf(qv[r][i], kv[st][i], p);
                p = sum8(p);
                if (jl < ncv && (lig & 7) == 0) s_lds[kvl * REP + r][st * GS + wslot] = p * a.scale;
            }
        }
        __syncthreads();
        if (tid < QH) {
            const int nv = min(SUB, ncv - sub);
            float mx = -INFINITY;
            for (int jl = 0; jl < nv; jl++) mx = fmaxf(mx, s_lds[tid][jl]);
            const float m_new = fmaxf(m_run, mx);
            const float alpha = expf(m_run - m_new);      // 0 on the first sub-step
            float sum = 0.f;
            for (int jl = 0; jl < nv; jl++) {
                float p = expf(s_lds[tid][jl] - m_new);
                s_lds[tid][jl] = p;
                sum += p;
            }
            l_run = l_run * alpha + sum;
            m_run = m_new;
            s_alpha[tid] = alpha;
        }
        __syncthreads();
#pragma unroll
        for (int r = 0; r < REP; r++) {
            const float al = s_alpha[kvl * REP + r];
#pragma unroll
            for (int i = 0; i < 8; i++) ov[r][i] *= al;
#pragma unroll
            for (int st = 0; st < NST; st++) {
                if (sub + st * GS + wslot < ncv) {
                    const float p = s_lds[kvl * REP + r][st * GS + wslot];
#pragma unroll
                    for (int i = 0; i < 8; i++) ov[r][i] = fmaf(p, vv[st][i], ov[r][i]);
                }
            }
        }
        __syncthreads();
    }
    // chunk partials
    if (tid < QH) {
        const int h = hg0 * REP + tid;
        a.ws_m[(int64_t)c * a.H + h] = m_run;
        a.ws_l[(int64_t)c * a.H + h] = l_run;
    }
#pragma unroll
    for (int r = 0; r < REP; r++)
#pragma unroll
        for (int i = 0; i < 8; i++) o_red[wslot * QH * DH + (kvl * REP + r) * DH + dim0 + i] = ov[r][i];
    __syncthreads();
    for (int e = tid; e < QH * DH; e += 256) {
        float acc = 0.f;
#pragma unroll
        for (int g = 0; g < GS; g++) acc += o_red[g * QH * DH + e];
        const int h = hg0 * REP + e / DH;
        a.ws_o[((int64_t)c * a.H + h) * DH + (e % DH)] = acc;
    }
    // ---- completion: the last chunk of this head group merges the partials
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    __syncthreads();
    const int nch = (L + CS - 1) / CS;
    if (tid == 0) {
        int prev = __hip_atomic_fetch_add(a.counters + blockIdx.y, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = (prev == nch - 1);
    }
    __syncthreads();
    if (!s_last) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    // per-head max and sum over chunks: QH heads x (256/QH) chunk lanes
    constexpr int CL = 256 / QH;
    float* wts = o_red;                                   // [nch][QH] softmax weights
    {
        const int hq = tid / CL, cl = tid % CL;
        const int h = hg0 * REP + hq;
        float mx = -INFINITY;
        for (int cc = cl; cc < nch; cc += CL) mx = fmaxf(mx, gld(a.ws_m + (int64_t)cc * a.H + h));
        o_red[GS * QH * DH - 256 + tid] = mx;
        __syncthreads();
        if (cl == 0) {
            float m = -INFINITY;
            for (int k = 0; k < CL; k++) m = fmaxf(m, o_red[GS * QH * DH - 256 + hq * CL + k]);
            s_hm[hq] = m;
        }
        __syncthreads();
        const float M = s_hm[hq];
        float ls = 0.f;
        for (int cc = cl; cc < nch; cc += CL) {
            float w = expf(gld(a.ws_m + (int64_t)cc * a.H + h) - M);
            wts[cc * QH + hq] = w;
            ls = fmaf(gld(a.ws_l + (int64_t)cc * a.H + h), w, ls);
        }
        o_red[GS * QH * DH - 256 + tid] = ls;
        __syncthreads();
        if (cl == 0) {
            float t = 0.f;
            for (int k = 0; k < CL; k++) t += o_red[GS * QH * DH - 256 + hq * CL + k];
            s_hl[hq] = 1.0f / t;
        }
        __syncthreads();
    }
    const int64_t cstride = (int64_t)a.H * DH;
    for (int e = tid; e < QH * DH; e += 256) {
        const int hq = e / DH, d = e % DH;
        const int h = hg0 * REP + hq;
        const float* op = a.ws_o + (int64_t)h * DH + d;
        float acc = 0.f;
        int cc = 0;
        for (; cc + 8 <= nch; cc += 8) {       // 8 independent loads in flight
            float o[8];
#pragma unroll
            for (int k = 0; k < 8; k++) o[k] = gld(op + (cc + k) * cstride);
#pragma unroll
            for (int k = 0; k < 8; k++) acc = fmaf(o[k], wts[(cc + k) * QH + hq], acc);
        }
        for (; cc < nch; cc++) acc = fmaf(gld(op + cc * cstride), wts[cc * QH + hq], acc);
        gst(a.out + (int64_t)h * DH + d, acc * s_hl[hq]);
    }
    if (tid == 0) __hip_atomic_store(a.counters + blockIdx.y, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// Generic causal kernel: any T, dh <= 256, pre-RoPE caches.  One wave per
// (query head, query row); keys in order with the online normalized update
// of flash_fp32.cu:55-81, parallel over dims.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float cache_val(int fmt, const uint8_t* c, int64_t idx) {
    if (fmt == 0) return ((const float*)c)[idx];
    return kvq::dequant_one(fmt, c + (idx >> 5) * kvq::block_bytes(fmt), (int)(idx & 31));
}

__global__ __launch_bounds__(64) void attn_generic_kernel(AttnArgs a, int kf, int vf) {
    const int h = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
    const int pos0 = read_pos(a.start_pos, a.d_pos);
    const int pq = pos0 + t;
    if (pos0 < 0 || pq >= a.max_seq) return;       // capacity guard
    const int dh = a.dh, half = dh / 2, kvd = a.Hkv * dh;
    const int kvh = h / (a.H / a.Hkv);
    float qv[4], ov[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        int d = lane + 64 * i;
        qv[i] = d < dh ? a.q[((int64_t)t * a.H + h) * dh + d] : 0.f;
        ov[i] = 0.f;
    }
    float m = -1e10f, l = 0.f, m_row = -1e10f;
    for (int j = 0; j <= pq; j++) {
        float kv[4], vv[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            int d = lane + 64 * i;
            kv[i] = vv[i] = 0.f;
            if (d >= dh) continue;
            if (j >= pos0) {
                kv[i] = a.kcur[(int64_t)(j - pos0) * kvd + kvh * dh + d];
                vv[i] = a.vcur[(int64_t)(j - pos0) * kvd + kvh * dh + d];
            } else {
                int64_t base = (int64_t)j * kvd + kvh * dh;
                float x = cache_val(kf, a.ck, base + d);
                if (a.pre_rope && a.rkc) {   // gqa_layer.cu:236-238: rotate cached raw K
                    int dp = d < half ? d + half : d - half;
                    float xp = cache_val(kf, a.ck, base + dp);
                    float cs = a.rkc[(int64_t)j * half + (d % half)], sn = a.rks[(int64_t)j * half + (d % half)];
                    x = d < half ? x * cs - xp * sn : xp * sn + x * cs;
                }
                kv[i] = x;
                vv[i] = cache_val(vf, a.cv, base + d);
            }
        }
        float p = 0.f;
#pragma unroll
        for (int i = 0; i < 4; i++) p = fmaf(qv[i], kv[i], p);
        float s = wave_sum(p) * a.scale;
        float old_l = l;
        float new_m = fmaxf(m, s);
        l = fmaf(l, expf(m - new_m), expf(s - new_m));
        m = new_m;
        float so = old_l * expf(m_row - m) / l;
        float sn = expf(s - m) / l;
#pragma unroll
        for (int i = 0; i < 4; i++) ov[i] = fmaf(ov[i], so, vv[i] * sn);
        m_row = m;
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        int d = lane + 64 * i;
        if (d < dh) a.out[((int64_t)t * a.H + h) * dh + d] = ov[i];
    }
}

template <int KF, int VF, int HG>
int launch_decode_rep(AttnArgs a, int rep, hipStream_t st) {
    // sub-step of this head-group size: 16 positions, 32 for single heads
    const int gran = HG >= 2 ? 16 : 32;
    a.chunk = chunk_len(a.max_seq, gran);
    const int max_pos = a.d_pos ? a.max_seq : a.start_pos + 1;
    a.nchunk_max = (max_pos + a.chunk - 1) / a.chunk;
    const size_t need = kCounterBytes + (size_t)a.nchunk_max * a.H * (2 + (size_t)a.dh) * sizeof(float);
    if (!a.ws || a.ws_bytes < need) return RINA_ERR_WORKSPACE;
    a.counters = (int*)a.ws;
    a.ws_m = (float*)((char*)a.ws + kCounterBytes);
    a.ws_l = a.ws_m + (size_t)a.nchunk_max * a.H;
    a.ws_o = a.ws_l + (size_t)a.nchunk_max * a.H;
    dim3 grid(a.nchunk_max, a.Hkv / HG);
    switch (rep) {
        case 1: hipLaunchKernelGGL((attn_decode_kernel<KF, VF, HG, 1>), grid, dim3(256), 0, st, a); break;
        case 2: hipLaunchKernelGGL((attn_decode_kernel<KF, VF, HG, 2>), grid, dim3(256), 0, st, a); break;
        case 4: hipLaunchKernelGGL((attn_decode_kernel<KF, VF, HG, 4>), grid, dim3(256), 0, st, a); break;
        case 8: hipLaunchKernelGGL((attn_decode_kernel<KF, VF, HG, 8>), grid, dim3(256), 0, st, a); break;
        default: return RINA_ERR_SHAPE;
    }
    return hipGetLastError() == hipSuccess ? RINA_OK : RINA_ERR_HIP;
}

// head-group size per mode: enough heads that a position's K record slice
// spans >= ~128 contiguous bytes
template <int KF, int VF>
int launch_decode(const AttnArgs& a, int rep, hipStream_t st) {
    constexpr int HGP = KF == 0 ? 2 : KF == RINA_KVF_Q8_0 ? 4 : 8;
    if (a.Hkv % HGP == 0) return launch_decode_rep<KF, VF, HGP>(a, rep, st);
    if (a.Hkv % 4 == 0 && HGP > 4) return launch_decode_rep<KF, VF, 4>(a, rep, st);
    if (a.Hkv % 2 == 0 && HGP > 2) return launch_decode_rep<KF, VF, 2>(a, rep, st);
    return launch_decode_rep<KF, VF, 1>(a, rep, st);
}


}  // namespace

extern "C" size_t rina_hip_gqa_attention_workspace(int T, int H, int dh, int max_pos) {
    (void)T;
    // granularity 16 gives the most chunks, an upper bound for every kernel shape
    size_t nch = (size_t)(max_pos + chunk_len(max_pos, 16) - 1) / chunk_len(max_pos, 16);
    return kCounterBytes + nch * H * (2 + (size_t)dh) * sizeof(float);
}

extern "C" int rina_hip_gqa_attention(const float* q, const float* kcur, const float* vcur, const void* cache_k,
                                      const void* cache_v, int mode, int pre_rope, const float* rkc, const float* rks,
                                      int T, int H, int Hkv, int dh, int start_pos, const int* d_pos, int max_seq,
                                      float* out, void* workspace, size_t ws_bytes, void* stream) {
    if (!q || !kcur || !vcur || !out || T < 1 || H < 1 || Hkv < 1 || dh < 1 || max_seq < 1) return RINA_ERR_ARG;
    if (mode < RINA_KV_FP32 || mode > RINA_KV_Q2K_Q1V) return RINA_ERR_QTYPE;
    if (H % Hkv || dh > 256) return RINA_ERR_SHAPE;
    if (mode != RINA_KV_FP32 && (Hkv * dh) % 32) return RINA_ERR_SHAPE;
    if (!d_pos && (start_pos < 0 || start_pos + T > max_seq)) return RINA_ERR_RANGE;
    bool need_cache = d_pos || start_pos > 0;
    if (need_cache && (!cache_k || !cache_v)) return RINA_ERR_ARG;
    hipStream_t st = as_stream(stream);
    int kf = 0, vf = 0;
    if (mode != RINA_KV_FP32) kvq::mode_formats_host(mode, kf, vf);
    AttnArgs a{};
    a.q = q; a.kcur = kcur; a.vcur = vcur;
    a.ck = (const uint8_t*)cache_k; a.cv = (const uint8_t*)cache_v;
    a.rkc = rkc; a.rks = rks; a.out = out;
    a.mode = mode; a.pre_rope = pre_rope; a.T = T; a.H = H; a.Hkv = Hkv; a.dh = dh;
    a.start_pos = start_pos; a.max_seq = max_seq; a.d_pos = d_pos;
    a.scale = 1.0f / sqrtf((float)dh);
    int rep = H / Hkv;
    bool fast = T == 1 && dh == 64 && !pre_rope && (rep == 1 || rep == 2 || rep == 4 || rep == 8) &&
                ((uintptr_t)q % 16 == 0) && ((uintptr_t)kcur % 16 == 0) && ((uintptr_t)vcur % 16 == 0) &&
                (mode != RINA_KV_FP32 || (((uintptr_t)cache_k | (uintptr_t)cache_v) % 16 == 0));
    if (fast) {
        a.ws = workspace;
        a.ws_bytes = ws_bytes;
        switch (mode) {
            case RINA_KV_FP32: return launch_decode<0, 0>(a, rep, st);
            case RINA_KV_Q8: return launch_decode<RINA_KVF_Q8_0, RINA_KVF_Q8_0>(a, rep, st);
            case RINA_KV_Q4: return launch_decode<RINA_KVF_Q4_0, RINA_KVF_Q4_0>(a, rep, st);
            case RINA_KV_Q4K_Q2V: return launch_decode<RINA_KVF_Q4_0, RINA_KVF_Q2_1>(a, rep, st);
            case RINA_KV_Q2: return launch_decode<RINA_KVF_Q2_1, RINA_KVF_Q2_1>(a, rep, st);
            default: return launch_decode<RINA_KVF_Q2_1, RINA_KVF_Q1_0>(a, rep, st);
        }
    }
    hipLaunchKernelGGL(attn_generic_kernel, dim3(H, T), dim3(64), 0, st, a, kf, vf);
    RINA_LAUNCH_CHECK();
    return RINA_OK;
}
