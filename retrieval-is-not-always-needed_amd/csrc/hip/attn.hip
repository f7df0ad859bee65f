// Single-layer GQA attention over the (quantized) KV cache.
//
// Semantics (rina-engine/src/arch/gqa/gqa_layer.cu:192-270 with
// kernels/flash_fp32.cu:12-111 and build_qkv_fp32.cu:8-33): query row t sits
// at position pos0+t and attends causally to keys 0..pos0+t; keys/values
// below pos0 come from the cache (dequantized with the block rules of
// kernels/quantize.cu), the others from the current fp32 rows; query head h
// reads KV head h / (H/Hkv); score = (q.k) / sqrt(dh).
//
// Decode (T == 1, dh == 64), fp32 cache of at most 1024 positions: one
// launch (attn_vsplit_kernel, below: every workgroup scores the whole
// context for one query head and keeps a slice of the value dims).
// Otherwise split-sequence in two launches.  The split
// kernel gives each workgroup a chunk of positions of HG KV heads (records of
// a position are contiguous: position-major, heads inside); 8 lanes cover one
// head's 64 dims (8 values per lane, dequantized in registers) and the REP
// query heads of that KV head are reduced with DPP inside the 8-lane group
// (with an even REP, two sets of four waves take the same positions and half
// the query heads each: a shorter chain per lane, two waves per SIMD).
// Every 8-lane slot keeps its own online softmax over the positions it takes
// (no barrier in the loop; the next positions' K/V loads are in flight while
// the current ones are consumed); the slots merge through one LDS exchange,
// and the chunk writes (max, sum, O) partials with the maxima in base-2 units
// (scores carry log2 e, weights are exp2 values).  The combine kernel merges
// the chunks of each head.  Optionally the split kernel also
// applies RoPE to q and the current k and appends K/V at the current position
// (the workgroup holding that position), replacing the separate append launch.
#include "rina_common.hpp"
#include "kv_formats.hpp"
#include <mutex>

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kMaxChunks = 64;  // chunk partials per head (chunk length adapts)

// Chunk length for a cache of max_pos positions: at most kMaxChunks
// partials per head, each a multiple of the workgroup step `gran`.
int chunk_len(int max_pos, int gran) {
    int per = (max_pos + kMaxChunks - 1) / kMaxChunks;
    per = (per + gran - 1) / gran * gran;
    return per < gran ? gran : per;
}

struct AttnArgs {
    const float* q;
    const float* kcur;
    const float* vcur;
    const uint8_t* ck;
    const uint8_t* cv;
    const float* rkc;
    const float* rks;
    float* out;
    int mode, pre_rope, T, H, Hkv, dh, start_pos, max_seq;
    const int* d_pos;
    float scale;
};

struct SplitArgs {
    const float* q;        // [H*64]; raw when the kernel applies RoPE
    const float* kcur;     // [Hkv*64]; raw when the kernel applies RoPE
    const float* vcur;     // [Hkv*64]
    const float *qc, *qs, *kc, *ks;   // RoPE tables [max_seq][32] (NULL: no rotation)
    uint8_t* ck;           // caches; written at pos0 when the kernel appends
    uint8_t* cv;
    float* k_rot_out;      // optional copy of the appended (rotated) fp32 K row
    float* ws_m;           // [nchunk][H]
    float* ws_l;           // [nchunk][H]
    float* ws_o;           // [nchunk][H][64]
    float* out;            // [H*64]
    int mode, H, Hkv, start_pos, max_seq, chunk;
    const int* d_pos;
    float scale;
};

typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));

// q8_0 slices in one load.  A lane's 8 values of a 34-byte block (scale,
// 32 codes) start at w = v0 % 32 in {0, 8, 16, 24}; with 2-byte aligned
// records the 12 bytes from the dword at or below block + w hold its codes
// at byte 2 + sh, sh = (block + w) % 4 in {0, 2}, and for w == 0 the block
// scale at byte sh.  The other lanes of the block (w 8, 16, 24: the next
// three lanes of the quad, by the kernels' lane layout) take the scale from
// the quad's first lane.  The window ends at most 2 bytes past the block
// (sh 0, w 24), inside the next block of the record or the next record: the
// callers read only records below the last one written (positions < pos0)
// or, for masked lanes, the query row (at least 4 * 64 bytes per KV head,
// more than the 68 of a q8 head-record).
__device__ __forceinline__ int q8_shift(const uint8_t* base, int64_t v0) {
    return (int)(((uintptr_t)(base + (v0 >> 5) * 34 + (v0 & 31))) & 3);
}
__device__ __forceinline__ u32x3 q8_window(const uint8_t* base, int64_t v0) {
    const uintptr_t st = (uintptr_t)(base + (v0 >> 5) * 34 + (v0 & 31));
    return gld((const u32x3*)(st & ~(uintptr_t)3));
}
// codes (as floats, exact) and the fp16 scale bits of a window
__device__ __forceinline__ uint32_t q8_unpack(const u32x3& x, int sh, float (&o)[8]) {
    const uint32_t lo = sh ? x.y : __builtin_amdgcn_alignbyte(x.y, x.x, 2);
    const uint32_t hi = sh ? x.z : __builtin_amdgcn_alignbyte(x.z, x.y, 2);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        o[i] = (float)(int8_t)(lo >> (8 * i));
        o[4 + i] = (float)(int8_t)(hi >> (8 * i));
    }
    const uint32_t own = (x.x >> (8 * sh)) & 0xFFFF;   // the scale in the w == 0 lane
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)own, 0x00, 0xf, 0xf, false);   // quad_perm [0,0,0,0]
}

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
    if (FMT == RINA_KVF_Q8_0) {
        const float s = f16_to_f32(q8_unpack(q8_window(base, v0), q8_shift(base, v0), o));
#pragma unroll
        for (int i = 0; i < 8; i++) o[i] *= s;
        return;
    }
    constexpr int BB = kvq::block_bytes_c(FMT);
    const uint8_t* blk = base + (v0 >> 5) * BB;
    const int w = (int)(v0 & 31);
    float s = f16_to_f32(gld((const uint16_t*)blk));
    if (FMT == RINA_KVF_Q4_0) {
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

// The raw words of load8's 8 values, loaded now and converted later by
// codes_raw8: loads can then be issued well before their values are needed
// without the conversion making the wave wait for them at issue.
struct Raw8 {
    float f[8];      // fp32 records
    u32x3 x;         // q8_0 records: the 12-byte window (q8_window)
    uint32_t h[4];   // other packed records: the 16-bit words load8 reads
    uint32_t s;      // other packed records: the fp16 scale
};

template <int FMT>
__device__ __forceinline__ void load_raw8(const uint8_t* base, int64_t v0, Raw8& r) {
    if (FMT == 0) {
        const f32x4* p = (const f32x4*)((const float*)base + v0);
        const f32x4 a = gld(p), b = gld(p + 1);
        r.f[0] = a.x; r.f[1] = a.y; r.f[2] = a.z; r.f[3] = a.w;
        r.f[4] = b.x; r.f[5] = b.y; r.f[6] = b.z; r.f[7] = b.w;
        return;
    }
    if (FMT == RINA_KVF_Q8_0) {
        r.x = q8_window(base, v0);
        return;
    }
    constexpr int BB = kvq::block_bytes_c(FMT);
    const uint8_t* blk = base + (v0 >> 5) * BB;
    const int w = (int)(v0 & 31);
    r.s = gld((const uint16_t*)blk);
    if (FMT == RINA_KVF_Q4_0) {
        r.h[0] = gld((const uint16_t*)(blk + 2 + w / 2));
        r.h[1] = gld((const uint16_t*)(blk + 4 + w / 2));
    } else if (FMT == RINA_KVF_Q2_1) {
        r.h[0] = gld((const uint16_t*)(blk + 2 + w / 4));
    } else {
        r.h[0] = gld((const uint16_t*)(blk + 2));
        r.h[1] = gld((const uint16_t*)(blk + 4));
    }
}

// The 8 values of a Raw8 as load8 would give them, without the block scale:
// the integer codes as floats (exact), the scale returned apart (1 for fp32
// records), so a consumer applies it once per lane instead of once per value
// (sh: q8_shift of the record's lane slice; q8_0 only)
template <int FMT>
__device__ __forceinline__ float codes_raw8(const Raw8& r, int64_t v0, int sh, float (&o)[8]) {
    if (FMT == 0) {
#pragma unroll
        for (int i = 0; i < 8; i++) o[i] = r.f[i];
        return 1.0f;
    }
    if (FMT == RINA_KVF_Q8_0) return f16_to_f32(q8_unpack(r.x, sh, o));
    const int w = (int)(v0 & 31);
    if (FMT == RINA_KVF_Q4_0) {
        const uint32_t n = r.h[0] | (r.h[1] << 16);
#pragma unroll
        for (int i = 0; i < 8; i++) o[i] = (float)((int)((n >> (4 * i)) & 0xF) - 7);
    } else if (FMT == RINA_KVF_Q2_1) {
        const uint32_t n = r.h[0];
#pragma unroll
        for (int i = 0; i < 8; i++) o[i] = (float)((int)((n >> (2 * i)) & 3) - 1);
    } else {
        const uint32_t bits = (r.h[0] | (r.h[1] << 16)) >> w;
#pragma unroll
        for (int i = 0; i < 8; i++) o[i] = ((bits >> i) & 1u) ? 1.0f : -1.0f;
    }
    return f16_to_f32(r.s);
}

__device__ __forceinline__ void ld8f(const float* p, float (&o)[8]) {
    const f32x4* v = (const f32x4*)p;
    f32x4 a = gld(v), b = gld(v + 1);
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
    o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
}

// Dims [dim0, dim0+8) of a 64-dim head row after the NeoX rotation with
// table row (c, s) (ops/rope.cu:125-149, same fused-multiply form as the
// reference's compiled kernel: x0*c - x1*s and x0*s + x1*c with one rounding
// of the x1 product inside each fma).  own: the row's values at these dims;
// pair: the values 32 dims away.
__device__ __forceinline__ void rope8(int dim0, const float (&own)[8], const float (&pair)[8], const float (&c)[8],
                                      const float (&s)[8], float (&o)[8]) {
    if (dim0 < 32) {
#pragma unroll
        for (int i = 0; i < 8; i++) o[i] = fmaf(own[i], c[i], -(pair[i] * s[i]));
    } else {
#pragma unroll
        for (int i = 0; i < 8; i++) o[i] = fmaf(pair[i], s[i], own[i] * c[i]);
    }
}

constexpr int kSplitEntrySteps = 5;   // steps a split workgroup loads at entry (80 positions)

template <int KF, int VF, int HG, int REP, bool FUSED, int QS>
__global__ __launch_bounds__(256 * QS) void attn_split_kernel(SplitArgs a) {
    constexpr int DH = 64;
    constexpr int LPP = 8 * HG;          // lanes per position record
    constexpr int PPW = 64 / LPP;        // positions per wave step (slots)
    constexpr int GS = 4 * PPW;          // positions per workgroup step
    constexpr int QH = HG * REP;         // query heads in the group
    constexpr int RL = REP / QS;         // query heads of a KV head per wave: QS wave sets
                                         // (waves 4 q .. 4 q + 3) share the positions
    constexpr int NS = 4 * PPW;          // softmax slots of the workgroup
    __shared__ __align__(16) float s_o[NS][QH][DH];
    __shared__ __align__(16) float s_m[QH][NS];
    __shared__ __align__(16) float s_aw[QH][NS];
    __shared__ float s_l[QH][NS], s_M[QH];
    __shared__ float s_k[FUSED ? HG * DH : 1], s_v[FUSED ? HG * DH : 1];

    const int tid = threadIdx.x, lane = tid & 63, wave = (tid >> 6) & 3, wq = tid >> 8;
    const int pos0 = read_pos(a.start_pos, a.d_pos);
    if (pos0 < 0 || pos0 >= a.max_seq) return;     // capacity guard (host checks host-known positions)
    const int L = pos0 + 1;
    const int CS = a.chunk;
    const int c = blockIdx.x;
    const int j0 = c * CS;
    if (j0 >= L) return;
    const int ncv = min(CS, L - j0);
    const bool has_cur = pos0 < j0 + CS;            // this chunk holds the current position
    const int kvd = a.Hkv * DH;
    const int hg0 = blockIdx.y * HG;
    constexpr int KBB = kvq::block_bytes_c(KF), VBB = kvq::block_bytes_c(VF);
    const int64_t KREC = KF ? (int64_t)(kvd / 32) * KBB : (int64_t)kvd * 4;
    const int64_t VREC = VF ? (int64_t)(kvd / 32) * VBB : (int64_t)kvd * 4;

    const int slot = lane / LPP, lig = lane % LPP;
    const int kvl = lig >> 3;                       // kv head inside the group
    const int dim0 = (lig & 7) * 8;
    const int kvh = hg0 + kvl;
    const int64_t voff = (int64_t)kvh * DH + dim0;  // value offset inside a position record
    const int wslot = wave * PPW + slot;

    // query rows (and the current K/V row) first: cache hits, rotated before
    // the chunk's K/V loads are issued.  The query-side loads sit under no
    // branch (without RoPE tables the query rows stand in for them, unused):
    // loads under a branch can leave register copies at the join that wait
    // for them there.  The current row is read by the workgroup that holds
    // it only (a uniform branch).
    float qraw[RL][8], qpair[RL][8], tc[8], ts[8];
    float kown[8], kpair[8], kc8[8], ks8[8], vcur[8];
    const bool qrope = FUSED && a.qc, krope = FUSED && a.kc;
    const int64_t toff = (int64_t)pos0 * 32 + (dim0 & 31);
#pragma unroll
    for (int r = 0; r < RL; r++) {
        const float* qh = a.q + (int64_t)(kvh * REP + wq * RL + r) * DH;
        ld8f(qh + dim0, qraw[r]);
        if constexpr (FUSED) ld8f(qh + (dim0 ^ 32), qpair[r]);
    }
    if constexpr (FUSED) {
        ld8f(qrope ? a.qc + toff : a.q, tc);
        ld8f(qrope ? a.qs + toff : a.q, ts);
    }
#pragma unroll
    for (int i = 0; i < 8; i++) kown[i] = vcur[i] = kpair[i] = kc8[i] = ks8[i] = 0.f;
    if (has_cur) {
        ld8f(a.kcur + voff, kown);
        ld8f(a.vcur + voff, vcur);
        if constexpr (FUSED) {
            ld8f(a.kcur + (int64_t)kvh * DH + (dim0 ^ 32), kpair);
            ld8f(krope ? a.kc + toff : a.kcur, kc8);
            ld8f(krope ? a.ks + toff : a.kcur, ks8);
        }
    }

    // K/V of step st: every lane loads, so the load counters stay exact
    // across the pipelined steps.  Lanes of positions past the chunk, and of
    // the current position (its rows come from kcur / vcur), read the query
    // row instead: in bounds, ignored, and no read reaches a cache record at
    // or past pos0 (the q8 windows may end 2 bytes into the next record).
    const int nsteps = (ncv + GS - 1) / GS;
    auto kv_rec = [&](int st, const uint8_t*& kb, const uint8_t*& vb) {
        const int jl = st * GS + wslot;
        const bool rd = jl < ncv && j0 + jl < pos0;
        kb = rd ? a.ck + (int64_t)(j0 + jl) * KREC : (const uint8_t*)a.q;
        vb = rd ? a.cv + (int64_t)(j0 + jl) * VREC : (const uint8_t*)a.q;
    };
    auto issue = [&](int st, float (&kk)[8], float (&vv)[8]) {
        const uint8_t *kb, *vb;
        kv_rec(st, kb, vb);
        load8<KF>(kb, voff, kk);
        load8<VF>(vb, voff, vv);
    };
    float kA[8], vA[8], kB[8], vB[8];
    // fp32 records with 4 query heads per wave: 3 entry steps (5 spill)
    constexpr int NE = (KF == 0 && VF == 0 && RL >= 4) ? 3 : kSplitEntrySteps;
    Raw8 kr[NE - 1], vr[NE - 1];
    // q8 windows: the lane's byte offset inside its dword (the same in every
    // record, whose length is a multiple of 4 bytes)
    const int ksh = KF == RINA_KVF_Q8_0 ? q8_shift(a.ck, voff) : 0;
    const int vsh = VF == RINA_KVF_Q8_0 ? q8_shift(a.cv, voff) : 0;

    // scores in base-2 units: log2 e and the scale folded into q, so the
    // softmax weights are hardware exp2 values
    float qv[RL][8];
    const float qsc = a.scale * 1.44269504088896341f;
#pragma unroll
    for (int r = 0; r < RL; r++) {
        if (qrope) rope8(dim0, qraw[r], qpair[r], tc, ts, qv[r]);
        else {
#pragma unroll
            for (int i = 0; i < 8; i++) qv[r][i] = qraw[r][i];
        }
#pragma unroll
        for (int i = 0; i < 8; i++) qv[r][i] *= qsc;
    }
    float kcur[8];                                  // used only where has_cur
    if (krope) rope8(dim0, kown, kpair, kc8, ks8, kcur);
    else {
#pragma unroll
        for (int i = 0; i < 8; i++) kcur[i] = kown[i];
    }

    float ov[RL][8], m_run[RL], l_run[RL];
#pragma unroll
    for (int r = 0; r < RL; r++) {
        m_run[r] = -INFINITY;
        l_run[r] = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) ov[r][i] = 0.f;
    }
    auto consume = [&](int st, const float (&kk)[8], const float (&vv)[8]) {
        const int jl = st * GS + wslot;
        const bool valid = jl < ncv;
        float kx[8], vx[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            kx[i] = kk[i];
            vx[i] = vv[i];
        }
        if (has_cur) {                              // uniform: the workgroup holding pos0
            const bool cur = j0 + jl == pos0;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                kx[i] = cur ? kcur[i] : kx[i];
                vx[i] = cur ? vcur[i] : vx[i];
            }
        }
#pragma unroll
        for (int r = 0; r < RL; r++) {
            float p = 0.f;
#pragma unroll
            for (int i = 0; i < 8; i++) p = fmaf(qv[r][i], kx[i], p);
            const float sc = sum8(p);
            if (valid) {
                const float mn = fmaxf(m_run[r], sc);
                const float al = __builtin_amdgcn_exp2f(m_run[r] - mn);   // 0 while nothing is accumulated
                const float pe = __builtin_amdgcn_exp2f(sc - mn);
                l_run[r] = fmaf(l_run[r], al, pe);
#pragma unroll
                for (int i = 0; i < 8; i++) ov[r][i] = fmaf(ov[r][i], al, pe * vx[i]);
                m_run[r] = mn;
            }
        }
    };
    // The first NE steps' loads are issued together, after the
    // query rotation (cache loads issued before it delay the query's round
    // trip, and with it the whole chain), every key first, then every value:
    // loads retire in issue order, so the scores wait for the keys alone.
    // Steps past 0 stay raw words until consumed.  Chunks of up to NE
    // steps then cost one memory round trip and run the
    // softmax scores first: every step's score (block scales applied once per
    // lane), one maximum per slot, then one exp2 and 8 FMAs per position, no
    // rescaling chain.  Longer chunks go on with one step in flight ahead of
    // the one consumed and the running softmax.  Measured at q8 (H 32 / Hkv
    // 8, 80-position chunks, split + combine per call, graph replay over 128
    // caches of 4104 positions, 572 MB): at positions 1000 / 2047 / 4095,
    // one step in flight 8.93 / 9.66 / 10.15 us, scores first 8.57 / 9.45 /
    // 9.81, these loads (12-byte q8 windows) 8.55 / 9.22 / 9.46.
    {
        const uint8_t *kb[NE], *vb[NE];
#pragma unroll
        for (int st = 0; st < NE; st++) kv_rec(st, kb[st], vb[st]);
        load8<KF>(kb[0], voff, kA);
#pragma unroll
        for (int st = 1; st < NE; st++) load_raw8<KF>(kb[st], voff, kr[st - 1]);
        load8<VF>(vb[0], voff, vA);
#pragma unroll
        for (int st = 1; st < NE; st++) load_raw8<VF>(vb[st], voff, vr[st - 1]);
    }
    if (nsteps <= NE) {
        // the current position's record replaces the cache's (uniform branch)
        auto is_cur = [&](int st) { return has_cur && j0 + st * GS + wslot == pos0; };
        float sc[NE][RL];
#pragma unroll
        for (int st = 0; st < NE; st++) {
#pragma unroll
            for (int r = 0; r < RL; r++) sc[st][r] = -INFINITY;
            if (st >= nsteps) continue;
            float kk[8];
            float ks = 1.0f;
            if (st == 0) {
#pragma unroll
                for (int i = 0; i < 8; i++) kk[i] = kA[i];
            } else {
                ks = codes_raw8<KF>(kr[st - 1], voff, ksh, kk);
            }
            if (has_cur) {
                const bool cur = is_cur(st);
#pragma unroll
                for (int i = 0; i < 8; i++) kk[i] = cur ? kcur[i] : kk[i];
                ks = cur ? 1.0f : ks;
            }
            const bool valid = st * GS + wslot < ncv;
#pragma unroll
            for (int r = 0; r < RL; r++) {
                float p = 0.f;
#pragma unroll
                for (int i = 0; i < 8; i++) p = fmaf(qv[r][i], kk[i], p);
                const float t = sum8(p * ks);
                sc[st][r] = valid ? t : -INFINITY;
            }
        }
#pragma unroll
        for (int r = 0; r < RL; r++) {
            float mx = sc[0][r];
#pragma unroll
            for (int st = 1; st < NE; st++) mx = fmaxf(mx, sc[st][r]);
            m_run[r] = mx;
        }
#pragma unroll
        for (int st = 0; st < NE; st++) {
            if (st >= nsteps) break;
            float vv[8];
            float vs = 1.0f;
            if (st == 0) {
#pragma unroll
                for (int i = 0; i < 8; i++) vv[i] = vA[i];
            } else {
                vs = codes_raw8<VF>(vr[st - 1], voff, vsh, vv);
            }
            if (has_cur) {
                const bool cur = is_cur(st);
#pragma unroll
                for (int i = 0; i < 8; i++) vv[i] = cur ? vcur[i] : vv[i];
                vs = cur ? 1.0f : vs;
            }
#pragma unroll
            for (int r = 0; r < RL; r++) {
                // masked positions (their records are not this step's and
                // may hold anything) add nothing; a slot with none valid
                // keeps m = -inf, l = 0, O = 0
                if (sc[st][r] != -INFINITY) {
                    const float pe = __builtin_amdgcn_exp2f(sc[st][r] - m_run[r]);
                    l_run[r] += pe;
                    const float pv = pe * vs;
#pragma unroll
                    for (int i = 0; i < 8; i++) ov[r][i] = fmaf(pv, vv[i], ov[r][i]);
                }
            }
        }
    } else {
        // the entry steps with the running softmax, step NE's loads in
        // flight meanwhile, then one step in flight ahead of the one consumed
        issue(NE, kB, vB);
        consume(0, kA, vA);
#pragma unroll
        for (int st = 1; st < NE; st++) {
            float kk[8], vv[8];
            const float ks = codes_raw8<KF>(kr[st - 1], voff, ksh, kk);
            const float vs = codes_raw8<VF>(vr[st - 1], voff, vsh, vv);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                kk[i] *= ks;
                vv[i] *= vs;
            }
            consume(st, kk, vv);
        }
        for (int st = NE;;) {
            if (st + 1 < nsteps) {
                issue(st + 1, kA, vA);
                consume(st, kB, vB);
            } else {
                consume(st, kB, vB);
                break;
            }
            st++;
            if (st + 1 < nsteps) {
                issue(st + 1, kB, vB);
                consume(st, kA, vA);
            } else {
                consume(st, kA, vA);
                break;
            }
            st++;
        }
    }

    // merge of the NS slots through LDS: every slot's (m, l, O) is written,
    // the slot weights 2^(m - M) are formed once per (head, slot), then each
    // output dim sums the weighted slots
    if ((lig & 7) == 0) {
#pragma unroll
        for (int r = 0; r < RL; r++) {
            s_m[kvl * REP + wq * RL + r][wslot] = m_run[r];
            s_l[kvl * REP + wq * RL + r][wslot] = l_run[r];
        }
    }
#pragma unroll
    for (int r = 0; r < RL; r++) {
        f32x4* dst = (f32x4*)&s_o[wslot][kvl * REP + wq * RL + r][dim0];
        dst[0] = f32x4{ov[r][0], ov[r][1], ov[r][2], ov[r][3]};
        dst[1] = f32x4{ov[r][4], ov[r][5], ov[r][6], ov[r][7]};
    }
    if (FUSED && has_cur && tid < LPP) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            s_k[kvl * DH + dim0 + i] = kcur[i];
            s_v[kvl * DH + dim0 + i] = vcur[i];
        }
    }
    __syncthreads();
    if (tid < QH * NS) {
        const int qh = tid / NS, sl = tid % NS;
        float M = -INFINITY;
#pragma unroll
        for (int k = 0; k < NS; k += 4) {
            const f32x4 mv = *(const f32x4*)&s_m[qh][k];
            M = fmaxf(fmaxf(M, fmaxf(mv.x, mv.y)), fmaxf(mv.z, mv.w));
        }
        const float mo = s_m[qh][sl];
        s_aw[qh][sl] = mo == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mo - M);
        if (sl == 0) s_M[qh] = M;
    }
    __syncthreads();
    for (int e = tid; e < QH * DH; e += 256 * QS) {
        const int qh = e / DH, d = e % DH;
        float o = 0.f;
#pragma unroll
        for (int k = 0; k < NS; k += 4) {
            const f32x4 w4 = *(const f32x4*)&s_aw[qh][k];
            o = fmaf(s_o[k][qh][d], w4.x, o);
            o = fmaf(s_o[k + 1][qh][d], w4.y, o);
            o = fmaf(s_o[k + 2][qh][d], w4.z, o);
            o = fmaf(s_o[k + 3][qh][d], w4.w, o);
        }
        const int h = hg0 * REP + qh;
        gst(a.ws_o + ((int64_t)c * a.H + h) * DH + d, o);
        if (d == 0) {
            float l = 0.f;
#pragma unroll
            for (int k = 0; k < NS; k++) l = fmaf(s_l[qh][k], s_aw[qh][k], l);
            gst(a.ws_m + (int64_t)c * a.H + h, s_M[qh]);
            gst(a.ws_l + (int64_t)c * a.H + h, l);
        }
    }
    // K/V append at pos0 (positions < pos0 are the only cache rows read by
    // this launch, so the write races with nothing)
    if (FUSED && has_cur) {
        const int64_t row = (int64_t)pos0 * kvd + (int64_t)hg0 * DH;
        if (a.mode == RINA_KV_FP32) {
            if (tid < HG * DH) {
                gst((float*)a.ck + row + tid, s_k[tid]);
                gst((float*)a.cv + row + tid, s_v[tid]);
            }
        } else if (tid < 2 * HG * DH) {
            // one value per thread, a half wave per 32-value block; K fills
            // the first HG*DH threads (whole waves), V the next
            const bool isv = tid >= HG * DH;
            const int e = isv ? tid - HG * DH : tid;
            const int64_t blk = row / 32 + e / 32;
            if (isv) kvq::quantize_block_lanes(VF, s_v[e], a.cv + blk * VBB);
            else kvq::quantize_block_lanes(KF, s_k[e], a.ck + blk * KBB);
        }
        if (a.k_rot_out && tid < HG * DH) gst(a.k_rot_out + (int64_t)hg0 * DH + tid, s_k[tid]);
    }
}

// ---------------------------------------------------------------------------
// Decode attention in one launch for fp32 caches of up to kVsMaxPos
// positions (pos0 < kVsMaxPos), dh == 64.  One workgroup per (query head,
// slice of 64/VS value dims): it scores every position of the context
// against the full 64-dim key rows of the head's KV head and accumulates
// only its value slice, so the VS workgroups of a head repeat the scores
// instead of exchanging partials, and the output is written normalized (no
// partials, no combine launch).  1024 threads: 4 lanes per position record
// (16 key dims and VD/4 value dims each), 256 positions per step, NST steps
// (the launch's position bound), every step's loads issued at entry.  All scores first, then the wave's maximum
// and weights; the sums of weights and weighted values are reduced over the
// lanes of each DPP row and the 64 row partials of the workgroup merge
// through LDS.  RoPE of q and of the current k (the reference's NeoX
// pairs, fused-multiply form) and the append at pos0 are fused; only
// positions < pos0 are read from the cache, so the append races with
// nothing.
// ---------------------------------------------------------------------------
constexpr int kVsSteps = 4;
constexpr int kVsMaxPos = 256 * kVsSteps;      // pos0 + 1 <= 1024

template <int VS, int NST>
__global__ __launch_bounds__(1024) void attn_vsplit_kernel(SplitArgs a) {
    constexpr int DH = 64, VD = DH / VS, VL = VD / 4;   // value dims per workgroup / per lane
    static_assert(VL >= 1 && VL <= 4 && VD % 4 == 0, "VS 2, 4 or 8");
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    __shared__ __align__(16) float s_q[DH];          // rotated query row, scaled to base-2 units
    __shared__ __align__(16) float s_k[DH], s_v[DH]; // the current (rotated) key row and value row
    __shared__ float s_pm[16], s_pl[64];             // per wave: maximum; per DPP row: sum of weights
    __shared__ float s_po[VD][64];                   // per DPP row: weighted value sums
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int pos0 = read_pos(a.start_pos, a.d_pos);
    if (pos0 < 0 || pos0 >= a.max_seq || pos0 >= 256 * NST) return;   // host checks host-known positions
    const int L = pos0 + 1;
    // workgroup = (KV head, query head of it, value slice), numbered
    // kvh + Hkv * (...): with 8 KV heads every workgroup of a KV head runs
    // on one XCD (workgroups go to the XCDs round-robin) and the head's key
    // rows come into its L2 once
    const int kvh = blockIdx.x % a.Hkv, rest = blockIdx.x / a.Hkv;
    const int vs = rest % VS, qh = kvh * (a.H / a.Hkv) + rest / VS;
    const int kvd = a.Hkv * DH;
    const int g = tid >> 2, qq = tid & 3;            // position within a step, quarter of the record
    const int v0 = vs * VD + VL * qq;                // this lane's first value dim
    // small loads first (query row, the current rows, RoPE tables: every
    // thread loads, indices clamped), then every step's key / value loads
    // (lanes of positions from pos0 on load nothing and hold zeros): loads
    // retire in issue order, so the rotation below waits for the small ones
    // alone
    const int pr = tid < DH * 3 ? tid / DH : 0, pd = tid % DH;
    const float* psrc = pr == 0 ? a.q + (int64_t)qh * DH : (pr == 1 ? a.kcur : a.vcur) + (int64_t)kvh * DH;
    const float* ptc = pr == 0 ? a.qc : a.kc;
    const float* pts = pr == 0 ? a.qs : a.ks;
    const bool prot = pr != 2 && ptc != nullptr;
    const float own = gld(psrc + pd), pair = gld(psrc + (pd ^ 32));
    const int64_t toff = (int64_t)pos0 * 32 + (pd & 31);
    const float pc = gld(prot ? ptc + toff : psrc), psn = gld(prot ? pts + toff : psrc);
    __builtin_amdgcn_sched_barrier(0);
    float kk[NST][16], vv[NST][VL];
#pragma unroll
    for (int t = 0; t < NST; t++) {
        const int p = g + 256 * t;
#pragma unroll
        for (int i = 0; i < 16; i++) kk[t][i] = 0.f;
#pragma unroll
        for (int i = 0; i < VL; i++) vv[t][i] = 0.f;
        if (p >= pos0) continue;                     // (measured: 7.36 -> 7.21 us at position 528)
        const int pp = p;
        const float* kr = (const float*)a.ck + (int64_t)pp * kvd + kvh * DH + 4 * qq;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const f32x4 w = gld((const f32x4*)(kr + 16 * i));
            kk[t][4 * i] = w.x; kk[t][4 * i + 1] = w.y; kk[t][4 * i + 2] = w.z; kk[t][4 * i + 3] = w.w;
        }
        const float* vr = (const float*)a.cv + (int64_t)pp * kvd + kvh * DH + v0;
        if constexpr (VL == 2) {
            const f32x2 w = gld((const f32x2*)vr);
            vv[t][0] = w.x; vv[t][1] = w.y;
        } else {
#pragma unroll
            for (int i = 0; i < VL; i++) vv[t][i] = gld(vr + i);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    if (tid < DH * 3) {
        float x = own;
        if (prot) x = pd < 32 ? fmaf(own, pc, -(pair * psn)) : fmaf(pair, psn, own * pc);
        if (pr == 0) s_q[pd] = x * (a.scale * 1.44269504088896341f);   // scores in base-2 units
        else if (pr == 1) s_k[pd] = x;
        else s_v[pd] = x;
    }
    __syncthreads();
    float qv[16];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const f32x4 w = *(const f32x4*)&s_q[16 * i + 4 * qq];
        qv[4 * i] = w.x; qv[4 * i + 1] = w.y; qv[4 * i + 2] = w.z; qv[4 * i + 3] = w.w;
    }
    // every score first (the lane group of a position holds it after the
    // quad sum), then the wave's maximum
    float sc[NST];
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < NST; t++) {
        sc[t] = -INFINITY;
        if (256 * t > pos0) continue;                // uniform: no position of this step is in the context
        const int p = g + 256 * t;
        if (p == pos0) {                             // the current position: its rows from LDS
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const f32x4 w = *(const f32x4*)&s_k[16 * i + 4 * qq];
                kk[t][4 * i] = w.x; kk[t][4 * i + 1] = w.y; kk[t][4 * i + 2] = w.z; kk[t][4 * i + 3] = w.w;
            }
#pragma unroll
            for (int i = 0; i < VL; i++) vv[t][i] = s_v[v0 + i];
        }
        float d = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) d = fmaf(qv[i], kk[t][i], d);
        d += dpp_f<0xB1>(d);                         // quad_perm [1,0,3,2]
        d += dpp_f<0x4E>(d);                         // quad_perm [2,3,0,1]
        if (p < L) { sc[t] = d; mx = fmaxf(mx, d); }
    }
    const float mw = wave_max(mx);                   // -inf: no position of this wave is in the context
    float l = 0.f, o[VL];
#pragma unroll
    for (int i = 0; i < VL; i++) o[i] = 0.f;
#pragma unroll
    for (int t = 0; t < NST; t++) {
        const float pe = sc[t] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(sc[t] - mw);
        l += pe;
#pragma unroll
        for (int i = 0; i < VL; i++) o[i] = fmaf(pe, vv[t][i], o[i]);
    }
    // sums over the 4 position groups of each DPP row that share this
    // lane's quarter (lanes qq, qq + 4, qq + 8, qq + 12 of the row)
    l += dpp_f<0x124>(l);                            // row_ror:4
    l += dpp_f<0x128>(l);                            // row_ror:8
#pragma unroll
    for (int i = 0; i < VL; i++) {
        o[i] += dpp_f<0x124>(o[i]);
        o[i] += dpp_f<0x128>(o[i]);
    }
    const int rw = wave * 4 + (lane >> 4);           // DPP row of the workgroup (64)
    if ((lane & 15) < 4) {
        if (qq == 0) s_pl[rw] = l;
#pragma unroll
        for (int i = 0; i < VL; i++) s_po[VL * qq + i][rw] = o[i];
    }
    if (lane == 0) s_pm[wave] = mw;
    __syncthreads();
    // merge of the 64 row partials: one wave per output value (lane = row)
    if (wave < VD) {
        const float m = s_pm[lane >> 2];
        const float M = wave_max(m);
        const float w = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - M);
        const float num = wave_sum(w * s_po[wave][lane]);
        const float den = wave_sum(w * s_pl[lane]);
        if (lane == 0) gst(a.out + (int64_t)qh * DH + vs * VD + wave, num / den);
    }
    // append at pos0 by one workgroup of the KV head
    if (rest == 0 && tid < DH) {
        const int64_t row = (int64_t)pos0 * kvd + (int64_t)kvh * DH;
        gst((float*)a.ck + row + tid, s_k[tid]);
        gst((float*)a.cv + row + tid, s_v[tid]);
        if (a.k_rot_out) gst(a.k_rot_out + (int64_t)kvh * DH + tid, s_k[tid]);
    }
}

// out[h] = sum_c e^(m_c - M) O_c / sum_c e^(m_c - M) l_c over the chunks that
// hold positions 0..pos0 (at most kMaxChunks = 64).  One workgroup per query
// head.  Every wave reads all chunk maxima and sums at once (lane c: chunk c)
// and each thread (chunk group g, dim d) issues its 16 O loads together, so
// the kernel costs one memory round trip.
__global__ __launch_bounds__(256) void attn_combine_kernel(SplitArgs a) {
    constexpr int DH = 64;
    constexpr int PER = kMaxChunks / 4;
    __shared__ float s_o[4][DH];
    const int pos0 = read_pos(a.start_pos, a.d_pos);
    if (pos0 < 0 || pos0 >= a.max_seq) return;
    const int nch = (pos0 + a.chunk) / a.chunk;     // chunks holding positions 0..pos0
    const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, g = tid >> 6;
    const int cl = lane < nch ? lane : nch - 1;
    const float mr = gld(a.ws_m + (int64_t)cl * a.H + h), lr = gld(a.ws_l + (int64_t)cl * a.H + h);
    float ov[PER];
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const int cc = min(g + 4 * k, nch - 1);
        ov[k] = gld(a.ws_o + ((int64_t)cc * a.H + h) * DH + lane);
    }
    const float ml = lane < nch ? mr : -INFINITY;
    const float M = wave_max(ml);
    const float wl = lane < nch ? __builtin_amdgcn_exp2f(ml - M) : 0.f;   // partial maxima in base-2 units
    const float lt = wave_sum(wl * lr);
    float o = 0.f;
#pragma unroll
    for (int k = 0; k < PER; k++) o = fmaf(ov[k], __shfl(wl, g + 4 * k), o);   // wl is 0 past nch
    s_o[g][lane] = o;
    __syncthreads();
    if (g == 0) gst(a.out + (int64_t)h * DH + lane, ((s_o[0][lane] + s_o[1][lane]) + (s_o[2][lane] + s_o[3][lane])) / lt);
}

// ---------------------------------------------------------------------------
// Decode attention with key width dq = da + db != value width dv = 64
// (RinaMLAImpl, arch/mla/rina_mla_layer.cu:78-86): query [qa | RoPE_hf(qb)],
// key [ka | RoPE_hf(kb)] per KV head, scale 1/sqrt(dq), fp32 caches
// [max_seq][Hkv][dq] / [max_seq][Hkv][dv].  The split kernel gives each
// workgroup 32 positions of one query head (8 per wave, loads issued
// together, lanes over dims); every workgroup rotates its query row itself
// (HF pairs 2i, 2i+1), the one holding the current position also forms the
// current K/V rows in registers and uses them for that position, and the
// first query head of each KV head there appends them to the caches (no
// workgroup of the launch reads that cache row).  It writes the same
// (m, l, O) partials as the GQA split kernel, so the same combine kernel
// finishes it.
// ---------------------------------------------------------------------------
struct DqArgs {
    const float *qa, *qb, *ka, *kb, *v;
    const float *qc, *qs, *kc, *ks;     // HF RoPE tables [max_seq][db/2] (NULL: none)
    float* ck;                          // fp32 cache: [max_seq][Hkv][dq]
    float* cv;                          // fp32 cache: [max_seq][Hkv][dv]
    uint8_t* ckq;                       // q2k_q1v: key content, q2_1 blocks [max_seq][Hkv][da/32]
    float* ckr;                         // q2k_q1v: key RoPE part, fp32 [max_seq][Hkv][db]
    uint8_t* cvq;                       // q2k_q1v: values, q1_0 records [max_seq][Hkv][dv/32]
    float* out;                         // dq_prompt_kv_kernel: [T][H][dv]
    int H, Hkv, da, db, dv, start_pos, max_seq;
    const int* d_pos;
    float scale;
};

// Dim `lane` (< 64) of a q2_1-packed 64-value row / a q1_0-packed 64-value
// row (two 32-value blocks each): kernels/quantize.cu:106-133, :160-185.
__device__ __forceinline__ float q2_1_dim(const uint8_t* row, int lane) {
    const uint8_t* b = row + (lane >> 5) * 10;
    const int i = lane & 31;
    const float s = f16_to_f32(kvq::ld16(b));
    return (float)((int)((b[2 + (i >> 2)] >> ((i & 3) * 2)) & 3) - 1) * s;
}
__device__ __forceinline__ float q1_0_dim(const uint8_t* row, int lane) {
    const uint8_t* b = row + (lane >> 5) * 6;
    const int i = lane & 31;
    const float s = f16_to_f32(kvq::ld16(b));
    const uint32_t half = kvq::ld16(b + 2 + ((i >> 4) << 1));
    return ((half >> (i & 15)) & 1u) ? s : -s;
}

constexpr int kDqChunk = 32;

// grid H + Hkv: workgroup h < H builds query h; the rest append KV head h - H
// Dim i (< da + db) of the row [xa | RoPE_hf(xb)] at position pos (tables
// [max_seq][db/2], NULL: no rotation), the rotation in the reference's
// fused-multiply form.  Every load is issued unconditionally (clamped
// indices) so the caller's load counters stay exact.
__device__ __forceinline__ float dq_dim(const float* xa, const float* xb, const float* tc, const float* ts, int da,
                                        int db, int pos, int i) {
    const int hb = db / 2;
    const int j = i - da, pi = j < 0 ? 0 : (j >> 1 < hb ? j >> 1 : hb - 1);
    const float va = gld(xa + (i < da ? i : da - 1));
    const float* xbb = db > 0 ? xb : xa;
    const float x0 = gld(xbb + (db > 0 ? 2 * pi : 0)), x1 = gld(xbb + (db > 0 ? 2 * pi + 1 : 0));
    const bool rot = tc != nullptr && db > 0;
    const float c = gld((rot ? tc : xbb) + (rot ? (int64_t)pos * hb + pi : 0));
    const float sn = gld((rot ? ts : xbb) + (rot ? (int64_t)pos * hb + pi : 0));
    const float cc = rot ? c : 1.0f, ss = rot ? sn : 0.0f;
    const float vb = (j & 1) ? fmaf(x0, ss, x1 * cc) : fmaf(x0, cc, -(x1 * ss));
    return i < da ? va : vb;
}

// A prompt's rows for the RINA-MLA attention over fp32 caches: grid
// (T, H + Hkv), one workgroup per (row, head).  Query heads: [qa | HF-RoPE(qb)]
// of row t at position t into q_full [T][H][da+db]; KV heads: the key row
// [ka | HF-RoPE(kb)] into k_full [T][Hkv][da+db] and the cache, the value
// row into the cache and, zero-padded to da + db, into v_full.  The rows
// are the ones the decode kernel appends (dq_dim).
__global__ __launch_bounds__(256) void dq_rows_kernel(DqArgs a, float* q_full, float* k_full, float* v_full) {
    const int i = threadIdx.x, t = blockIdx.x, y = blockIdx.y;
    const int dq = a.da + a.db;
    if (i >= dq) return;
    if (y < a.H) {
        const float* qa = a.qa + ((int64_t)t * a.H + y) * a.da;
        const float* qb = a.qb + ((int64_t)t * a.H + y) * a.db;
        gst(q_full + ((int64_t)t * a.H + y) * dq + i, dq_dim(qa, qb, a.qc, a.qs, a.da, a.db, t, i));
        return;
    }
    const int kvh = y - a.H;
    const float* ka = a.ka + ((int64_t)t * a.Hkv + kvh) * a.da;
    const float* kb = a.kb + ((int64_t)t * a.Hkv + kvh) * a.db;
    const float kv = dq_dim(ka, kb, a.kc, a.ks, a.da, a.db, t, i);
    const int64_t o = ((int64_t)t * a.Hkv + kvh) * dq + i;
    gst(k_full + o, kv);
    gst(a.ck + o, kv);
    const float vv = i < a.dv ? gld(a.v + ((int64_t)t * a.Hkv + kvh) * a.dv + i) : 0.f;
    gst(v_full + o, vv);
    if (i < a.dv) gst(a.cv + ((int64_t)t * a.Hkv + kvh) * a.dv + i, vv);
}

// QKV: 0 = fp32 caches; 1 = the q2k_q1v cache (key content q2_1, key RoPE
// part fp32, values q1_0; da == 64, dv == 64)
template <int QKV>
__global__ __launch_bounds__(256) void dq_split_kernel(DqArgs a, SplitArgs p) {
    __shared__ float s_o[4][64];
    __shared__ float s_m[4], s_l[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int pos0 = read_pos(a.start_pos, a.d_pos);
    if (pos0 < 0 || pos0 >= a.max_seq) return;
    const int L = pos0 + 1, c = blockIdx.x, h = blockIdx.y;
    const int j0 = c * kDqChunk;
    if (j0 >= L) return;
    const int ncv = min(kDqChunk, L - j0);
    const int dq = a.da + a.db, rep = a.H / a.Hkv, kvh = h / rep;
    const bool has_cur = pos0 < j0 + kDqChunk;      // this chunk holds the current position
    // the rotated query row and the current key / value rows (dims lane,
    // lane + 64; the key row is used in the chunk holding pos0), before the
    // cache loads
    const int i1 = lane + 64 < dq ? lane + 64 : dq - 1;
    const float* qa = a.qa + (int64_t)h * a.da;
    const float* qb = a.qb + (int64_t)h * a.db;
    const bool hi = lane + 64 < dq;
    const float* ka = a.ka + (int64_t)kvh * a.da;
    const float* kb = a.kb + (int64_t)kvh * a.db;
    const float q0 = dq_dim(qa, qb, a.qc, a.qs, a.da, a.db, pos0, lane);
    const float q1v = dq_dim(qa, qb, a.qc, a.qs, a.da, a.db, pos0, i1);
    const float kc0 = dq_dim(ka, kb, a.kc, a.ks, a.da, a.db, pos0, lane);
    const float kc1v = dq_dim(ka, kb, a.kc, a.ks, a.da, a.db, pos0, i1);
    const float vc = gld(a.v + (int64_t)kvh * a.dv + lane);
    const float q1 = hi ? q1v : 0.f, kc1 = hi ? kc1v : 0.f;
    constexpr int PW = kDqChunk / 4;
    float k0[PW], k1[PW], vv[PW];
#pragma unroll
    for (int i = 0; i < PW; i++) {
        const int pp = wave + 4 * i;
        const int64_t jp = j0 + (pp < ncv ? pp : 0);
        if (QKV == 0) {
            const float* kr = a.ck + (jp * a.Hkv + kvh) * dq;
            k0[i] = gld(kr + lane);
            k1[i] = lane + 64 < dq ? gld(kr + lane + 64) : 0.f;
            vv[i] = gld(a.cv + (jp * a.Hkv + kvh) * a.dv + lane);
        } else {
            k0[i] = q2_1_dim(a.ckq + (jp * a.Hkv + kvh) * 20, lane);
            k1[i] = lane < a.db ? gld(a.ckr + (jp * a.Hkv + kvh) * a.db + lane) : 0.f;
            vv[i] = q1_0_dim(a.cvq + (jp * a.Hkv + kvh) * 12, lane);
        }
    }
    // scores in base-2 units (the partials the combine kernel merges)
    const float sc2 = a.scale * 1.44269504088896341f;
    float m = -INFINITY, l = 0.f, o = 0.f;
#pragma unroll
    for (int i = 0; i < PW; i++) {
        const bool cur = has_cur && j0 + wave + 4 * i == pos0;   // wave-uniform
        const float kk0 = cur ? kc0 : k0[i], kk1 = cur ? kc1 : k1[i], vx = cur ? vc : vv[i];
        const float sc = wave_sum(fmaf(q0, kk0, q1 * kk1)) * sc2;
        if (wave + 4 * i < ncv) {
            const float mn = fmaxf(m, sc);
            const float al = __builtin_amdgcn_exp2f(m - mn), pe = __builtin_amdgcn_exp2f(sc - mn);
            l = fmaf(l, al, pe);
            o = fmaf(o, al, pe * vx);
            m = mn;
        }
    }
    // append at pos0 by the KV head's first query head (no workgroup of
    // this launch reads that row)
    if (QKV == 0 && has_cur && h % rep == 0 && wave == 0) {
        float* kd = a.ck + ((int64_t)pos0 * a.Hkv + kvh) * dq;
        gst(kd + lane, kc0);
        if (lane + 64 < dq) gst(kd + lane + 64, kc1);
        gst(a.cv + ((int64_t)pos0 * a.Hkv + kvh) * a.dv + lane, vc);
    }
    if (QKV == 1 && has_cur && h % rep == 0) {
        // the current key content and value rows packed with the KV cache's
        // block codec (the same bytes as rina_hip_kv_quantize), the RoPE part
        // stored as is; lane d of wave 0 holds dim d of both rows, a half
        // wave per 32-value block
        if (wave == 0) {
            const int b = lane >> 5;
            if (lane < a.db) gst(a.ckr + ((int64_t)pos0 * a.Hkv + kvh) * a.db + lane, kc1);
            kvq::quantize_block_lanes(RINA_KVF_Q2_1, kc0, a.ckq + ((int64_t)pos0 * a.Hkv + kvh) * 20 + 10 * b);
            kvq::quantize_block_lanes(RINA_KVF_Q1_0, vc, a.cvq + ((int64_t)pos0 * a.Hkv + kvh) * 12 + 6 * b);
        }
    }
    s_o[wave][lane] = o;
    if (lane == 0) { s_m[wave] = m; s_l[wave] = l; }
    __syncthreads();
    if (wave == 0) {
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < 4; w++) M = fmaxf(M, s_m[w]);
        float ot = 0.f, lt = 0.f;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const float aw = s_m[w] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(s_m[w] - M);
            ot = fmaf(s_o[w][lane], aw, ot);
            lt = fmaf(s_l[w], aw, lt);
        }
        gst(p.ws_o + ((int64_t)c * a.H + h) * 64 + lane, ot);
        if (lane == 0) {
            gst(p.ws_m + (int64_t)c * a.H + h, M);
            gst(p.ws_l + (int64_t)c * a.H + h, lt);
        }
    }
}

// A prompt's T rows (rows at positions start_pos + t) over the fp32 caches
// (QKV 0) or the q2k_q1v cache (QKV 1).  dq_pack_rows_kernel, grid (T, Hkv),
// one wave per (row, KV head): the row's key and value as
// dq_split_kernel<QKV> appends them at its position (the same dims, lanes
// and, packed, block codec).  dq_prompt_kv_kernel, grid (T, H), four waves
// per (row, query head), after it: row t reads the positions before it from
// the cache (as dq_split_kernel<QKV> reads them) and its own position from
// its fp32 rows, as the decode step of that row would; each wave takes every
// fourth position of each 32-position chunk with the running softmax (the
// next chunk's loads issued before the current chunk is scored), then the
// four waves merge and the row is normalized.
template <int QKV>
__global__ __launch_bounds__(64) void dq_pack_rows_kernel(DqArgs a) {
    const int lane = threadIdx.x, t = blockIdx.x, kvh = blockIdx.y;
    const int pos = a.start_pos + t, dq = a.da + a.db;
    const int i1 = lane + 64 < dq ? lane + 64 : dq - 1;
    const float* ka = a.ka + ((int64_t)t * a.Hkv + kvh) * a.da;
    const float* kb = a.kb + ((int64_t)t * a.Hkv + kvh) * a.db;
    const float kc0 = dq_dim(ka, kb, a.kc, a.ks, a.da, a.db, pos, lane);
    const float kc1 = dq_dim(ka, kb, a.kc, a.ks, a.da, a.db, pos, i1);
    const float vc = gld(a.v + ((int64_t)t * a.Hkv + kvh) * a.dv + lane);
    const int64_t row = (int64_t)pos * a.Hkv + kvh;
    if (QKV == 0) {
        float* kd = a.ck + row * dq;
        gst(kd + lane, kc0);
        if (lane + 64 < dq) gst(kd + lane + 64, kc1);
        gst(a.cv + row * a.dv + lane, vc);
    } else {
        const int b = lane >> 5;
        if (lane < a.db) gst(a.ckr + row * a.db + lane, kc1);
        kvq::quantize_block_lanes(RINA_KVF_Q2_1, kc0, a.ckq + row * 20 + 10 * b);
        kvq::quantize_block_lanes(RINA_KVF_Q1_0, vc, a.cvq + row * 12 + 6 * b);
    }
}

template <int QKV>
__global__ __launch_bounds__(256) void dq_prompt_kv_kernel(DqArgs a) {
    constexpr int PW = kDqChunk / 4;
    __shared__ float s_o[4][64];
    __shared__ float s_m[4], s_l[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int t = blockIdx.x, h = blockIdx.y;
    const int pos0 = a.start_pos + t, L = pos0 + 1;
    const int dq = a.da + a.db, kvh = h / (a.H / a.Hkv);
    const int i1 = lane + 64 < dq ? lane + 64 : dq - 1;
    const bool hi = lane + 64 < dq;
    const float* qa = a.qa + ((int64_t)t * a.H + h) * a.da;
    const float* qb = a.qb + ((int64_t)t * a.H + h) * a.db;
    const float* ka = a.ka + ((int64_t)t * a.Hkv + kvh) * a.da;
    const float* kb = a.kb + ((int64_t)t * a.Hkv + kvh) * a.db;
    const float q0 = dq_dim(qa, qb, a.qc, a.qs, a.da, a.db, pos0, lane);
    const float q1v = dq_dim(qa, qb, a.qc, a.qs, a.da, a.db, pos0, i1);
    const float kc0 = dq_dim(ka, kb, a.kc, a.ks, a.da, a.db, pos0, lane);
    const float kc1v = dq_dim(ka, kb, a.kc, a.ks, a.da, a.db, pos0, i1);
    const float vc = gld(a.v + ((int64_t)t * a.Hkv + kvh) * a.dv + lane);
    const float q1 = hi ? q1v : 0.f, kc1 = hi ? kc1v : 0.f;
    // the wave's positions j0 + wave + 4 i of a chunk; positions at or past
    // pos0 read position 0's record (in the cache, never used)
    auto load = [&](int j0, float (&x0)[PW], float (&x1)[PW], float (&xv)[PW]) {
#pragma unroll
        for (int i = 0; i < PW; i++) {
            const int p = j0 + wave + 4 * i;
            const int64_t r = (int64_t)(p < pos0 ? p : 0) * a.Hkv + kvh;
            if (QKV == 0) {
                x0[i] = gld(a.ck + r * dq + lane);
                x1[i] = lane + 64 < dq ? gld(a.ck + r * dq + lane + 64) : 0.f;
                xv[i] = gld(a.cv + r * a.dv + lane);
            } else {
                x0[i] = q2_1_dim(a.ckq + r * 20, lane);
                x1[i] = lane < a.db ? gld(a.ckr + r * a.db + lane) : 0.f;
                xv[i] = q1_0_dim(a.cvq + r * 12, lane);
            }
        }
    };
    const float sc2 = a.scale * 1.44269504088896341f;   // scores in base-2 units
    float m = -INFINITY, l = 0.f, o = 0.f;
    auto consume = [&](int j0, const float (&x0)[PW], const float (&x1)[PW], const float (&xv)[PW]) {
#pragma unroll
        for (int i = 0; i < PW; i++) {
            const int p = j0 + wave + 4 * i;
            const bool cur = p == pos0;                  // wave-uniform
            const float kk0 = cur ? kc0 : x0[i], kk1 = cur ? kc1 : x1[i], vx = cur ? vc : xv[i];
            const float sc = wave_sum(fmaf(q0, kk0, q1 * kk1)) * sc2;
            if (p < L) {
                const float mn = fmaxf(m, sc);
                const float al = __builtin_amdgcn_exp2f(m - mn), pe = __builtin_amdgcn_exp2f(sc - mn);
                l = fmaf(l, al, pe);
                o = fmaf(o, al, pe * vx);
                m = mn;
            }
        }
    };
    float kA[PW], rA[PW], vA[PW], kB[PW], rB[PW], vB[PW];
    load(0, kA, rA, vA);
    for (int j0 = 0;;) {
        if (j0 + kDqChunk < L) {
            load(j0 + kDqChunk, kB, rB, vB);
            consume(j0, kA, rA, vA);
        } else {
            consume(j0, kA, rA, vA);
            break;
        }
        j0 += kDqChunk;
        if (j0 + kDqChunk < L) {
            load(j0 + kDqChunk, kA, rA, vA);
            consume(j0, kB, rB, vB);
        } else {
            consume(j0, kB, rB, vB);
            break;
        }
        j0 += kDqChunk;
    }
    s_o[wave][lane] = o;
    if (lane == 0) { s_m[wave] = m; s_l[wave] = l; }
    __syncthreads();
    if (wave == 0) {
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < 4; w++) M = fmaxf(M, s_m[w]);
        float ot = 0.f, lt = 0.f;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const float aw = s_m[w] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(s_m[w] - M);
            ot = fmaf(s_o[w][lane], aw, ot);
            lt = fmaf(s_l[w], aw, lt);
        }
        gst(a.out + ((int64_t)t * a.H + h) * 64 + lane, ot / lt);   // pos0 itself is always counted: lt > 0
    }
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

// Prompt attention from position 0 (every key and value is a current row,
// dh == 64): one wave per (query head, 16 query rows).  Keys and values
// come in blocks of 64 positions: lane j holds key j of the block (64
// floats) and lane d holds dim d of the block's 64 values, so a query's 64
// scores are one FMA chain per lane (the query from LDS, broadcast) and its
// output update is one FMA chain per lane (the weights from LDS, broadcast).
// Softmax per block in base-2 units (scale and log2 e folded into the
// query): one maximum and one rescale per query and block.  Causal: query
// row t sees positions 0..t.
constexpr int kPromptRows = 16;

__global__ __launch_bounds__(64) void attn_prompt_kernel(AttnArgs a) {
    constexpr int DH = 64;
    __shared__ __align__(16) float s_q[kPromptRows][DH];
    __shared__ __align__(16) float s_o[kPromptRows][DH];
    __shared__ float s_m[kPromptRows], s_l[kPromptRows];
    __shared__ __align__(16) float s_p[DH];
    const int h = blockIdx.x, lane = threadIdx.x;
    const int t0 = blockIdx.y * kPromptRows;
    const int nq = min(kPromptRows, a.T - t0);
    const int kvd = a.Hkv * DH, kvh = h / (a.H / a.Hkv);
    const float qsc = a.scale * 1.44269504088896341f;
    for (int i = 0; i < nq; i++) {
        s_q[i][lane] = a.q[((int64_t)(t0 + i) * a.H + h) * DH + lane] * qsc;
        s_o[i][lane] = 0.f;
    }
    if (lane < kPromptRows) {
        s_m[lane] = -INFINITY;
        s_l[lane] = 0.f;
    }
    const int tmax = t0 + nq - 1;
    for (int j0 = 0; j0 <= tmax; j0 += 64) {
        // key j0 + lane (clamped past tmax: masked below) and value dim lane
        const int jk = min(j0 + lane, tmax);
        const f32x4* kp = (const f32x4*)(a.kcur + (int64_t)jk * kvd + kvh * DH);
        float kr[DH];
#pragma unroll
        for (int i = 0; i < DH / 4; i++) {
            const f32x4 v = gld(kp + i);
            kr[4 * i] = v.x; kr[4 * i + 1] = v.y; kr[4 * i + 2] = v.z; kr[4 * i + 3] = v.w;
        }
        float vr[64];
#pragma unroll
        for (int j = 0; j < 64; j++) vr[j] = gld(a.vcur + (int64_t)min(j0 + j, tmax) * kvd + kvh * DH + lane);
        const int i0 = j0 > t0 ? j0 - t0 : 0;                  // rows before j0 see nothing of this block
#pragma unroll 1
        for (int i = i0; i < nq; i++) {
            const int t = t0 + i;
            float sc = 0.f;
#pragma unroll
            for (int d = 0; d < DH; d += 4) {
                const f32x4 qv = *(const f32x4*)&s_q[i][d];
                sc = fmaf(qv.x, kr[d], sc);
                sc = fmaf(qv.y, kr[d + 1], sc);
                sc = fmaf(qv.z, kr[d + 2], sc);
                sc = fmaf(qv.w, kr[d + 3], sc);
            }
            if (j0 + lane > t) sc = -INFINITY;
            const float mo = s_m[i];
            const float mn = fmaxf(mo, wave_max(sc));           // finite: position j0 <= t is in the block
            const float al = __builtin_amdgcn_exp2f(mo - mn);
            const float p = __builtin_amdgcn_exp2f(sc - mn);
            const float ls = wave_sum(p);
            s_p[lane] = p;
            float acc = 0.f;
#pragma unroll
            for (int j = 0; j < 64; j += 4) {
                const f32x4 pv = *(const f32x4*)&s_p[j];
                acc = fmaf(pv.x, vr[j], acc);
                acc = fmaf(pv.y, vr[j + 1], acc);
                acc = fmaf(pv.z, vr[j + 2], acc);
                acc = fmaf(pv.w, vr[j + 3], acc);
            }
            s_o[i][lane] = fmaf(s_o[i][lane], al, acc);
            if (lane == 0) {
                s_m[i] = mn;
                s_l[i] = fmaf(s_l[i], al, ls);
            }
        }
    }
    for (int i = 0; i < nq; i++) a.out[((int64_t)(t0 + i) * a.H + h) * DH + lane] = s_o[i][lane] / s_l[i];
}

// The same prompt attention on the matrix cores (v_mfma_f32_16x16x4f32: fp32
// products, fp32 sums), for query heads in groups of 4 that share a KV head
// (H / Hkv a multiple of 4).  A workgroup takes one group and 16 query rows
// with NSET sets of 4 waves, wave w of a set query head 4 blockIdx.x + w:
// set k takes the 64-position K/V blocks k, k + NSET, ..., each with its
// own online softmax, merged at the end through LDS (so the longest row
// tiles take 1 / NSET as many steps; launched with two sets, four measured
// slower).  A set stages its block once in LDS (the
// next block's loads in registers while the current one is multiplied).
// Per block a wave forms S^T = K Q^T (4 tiles of 16 keys x 16 rows, 16 steps
// of 4 dims each: lane l's A value is key l % 16 of the tile at dim
// 16 (l / 16) + step, its B value the query row l % 16 at that dim), so a
// lane holds 16 scores of one query row (keys 16 kt + 4 (l / 16) + e), the
// row maximum and sum take two cross-lane steps, and those scores are
// directly the B operand of O^T += V^T P^T (step 4 kt + e uses key
// 16 kt + 4 (l / 16) + e; A value: dim 4 (l % 16) + dt of that key for
// output tile dt).  A lane ends with dims 16 (l / 16) .. + 15 of its row.
// Base-2 softmax units and the per-block rescale as in attn_prompt_kernel.
template <int NSET>
__global__ __launch_bounds__(256 * NSET) void attn_prompt_mfma_kernel(AttnArgs a) {
    constexpr int DH = 64, LDK = DH + 4;
    __shared__ __align__(16) float s_k[NSET][64][LDK];
    __shared__ __align__(16) float s_v[NSET][64][LDK];
    const int tid = threadIdx.x, lane = tid & 63;
    const int ws = __builtin_amdgcn_readfirstlane(tid >> 8);     // wave set: even / odd blocks
    const int ts = tid & 255;
    const int w = __builtin_amdgcn_readfirstlane((tid >> 6) & 3);
    const int ntile = (a.T + kPromptRows - 1) / kPromptRows;
    const int t0 = (ntile - 1 - (int)blockIdx.y) * kPromptRows;   // longest row tiles first
    const int h = 4 * (int)blockIdx.x + w;
    const int kvh = 4 * (int)blockIdx.x / (a.H / a.Hkv);
    const int kvd = a.Hkv * DH;
    const int tmax = min(t0 + kPromptRows, a.T) - 1;
    const int nblk = tmax / 64 + 1, npair = (nblk + NSET - 1) / NSET;
    const int fr = lane & 15, g = lane >> 4;
    const int row = t0 + fr;
    const float qsc = a.scale * 1.44269504088896341f;
    float qv[16];                                   // row fr (clamped), dims 16 g .. 16 g + 15
    {
        const f32x4* qp = (const f32x4*)(a.q + ((int64_t)min(row, a.T - 1) * a.H + h) * DH + 16 * g);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const f32x4 v = gld(qp + i);
            qv[4 * i] = v.x * qsc; qv[4 * i + 1] = v.y * qsc; qv[4 * i + 2] = v.z * qsc; qv[4 * i + 3] = v.w * qsc;
        }
    }
    // staging: thread ts of a set moves dims 16 (ts % 4) .. + 15 of key
    // j0 + ts / 4 (clamped to tmax: such keys are masked)
    const int sk = ts >> 2, sq = ts & 3;
    f32x4 kr[4], vr[4];
    auto load_blk = [&](int j0) {
        const int64_t off = (int64_t)min(j0 + sk, tmax) * kvd + kvh * DH + 16 * sq;
        const f32x4* kp = (const f32x4*)(a.kcur + off);
        const f32x4* vp = (const f32x4*)(a.vcur + off);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            kr[i] = gld(kp + i);
            vr[i] = gld(vp + i);
        }
    };
    f32x4 o[4];                                     // O^T tile dt: dims 16 g + 4 e + dt of row fr
#pragma unroll
    for (int dt = 0; dt < 4; dt++) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, l = 0.f;
    load_blk(64 * ws);
    for (int ip = 0; ip < npair; ip++) {
        const int j0 = 64 * (NSET * ip + ws);       // this set's block; past tmax: none (same for the set)
        __syncthreads();                            // the previous block's operands are read
#pragma unroll
        for (int i = 0; i < 4; i++) {
            *(f32x4*)&s_k[ws][sk][16 * sq + 4 * i] = kr[i];
            *(f32x4*)&s_v[ws][sk][16 * sq + 4 * i] = vr[i];
        }
        __syncthreads();
        load_blk(j0 + 64 * NSET <= tmax ? j0 + 64 * NSET : j0);   // unconditional: the last block reloads itself
        if (j0 > tmax) continue;
        f32x4 s[4];
#pragma unroll
        for (int kt = 0; kt < 4; kt++) s[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int q4 = 0; q4 < 4; q4++) {
            f32x4 kv[4];
#pragma unroll
            for (int kt = 0; kt < 4; kt++) kv[kt] = *(const f32x4*)&s_k[ws][16 * kt + fr][16 * g + 4 * q4];
#pragma unroll
            for (int c = 0; c < 4; c++)
#pragma unroll
                for (int kt = 0; kt < 4; kt++)
                    s[kt] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[kt][c], qv[4 * q4 + c], s[kt], 0, 0, 0);
        }
        // causal mask, then the row's maximum over the lanes l % 16 == fr
        float mx = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 4; kt++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                if (j0 + 16 * kt + 4 * g + e > row) s[kt][e] = -INFINITY;
                mx = fmaxf(mx, s[kt][e]);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float mn = fmaxf(m, mx);              // finite: key j0 <= every row of the tile
        const float al = __builtin_amdgcn_exp2f(m - mn);
        float ps = 0.f;
#pragma unroll
        for (int kt = 0; kt < 4; kt++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                s[kt][e] = __builtin_amdgcn_exp2f(s[kt][e] - mn);
                ps += s[kt][e];
            }
        ps += __shfl_xor(ps, 16);
        ps += __shfl_xor(ps, 32);
        l = fmaf(l, al, ps);
        m = mn;
#pragma unroll
        for (int dt = 0; dt < 4; dt++) o[dt] *= al;
#pragma unroll
        for (int kt = 0; kt < 4; kt++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const f32x4 vv = *(const f32x4*)&s_v[ws][16 * kt + 4 * g + e][4 * fr];
#pragma unroll
                for (int dt = 0; dt < 4; dt++) o[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[dt], s[kt][e], o[dt], 0, 0, 0);
            }
    }
    // merge: set 1 leaves (m, l, O) in LDS, set 0 combines (set 0 always
    // holds block 0, so its maximum is finite; set 1's may be -inf: weight 0)
    __syncthreads();
    float* xch = &s_k[0][0][0];                     // 18 floats per thread of sets 1 ..
    if (ws > 0) {
        float* d = xch + 18 * (256 * (ws - 1) + ts);
        d[0] = m;
        d[1] = l;
#pragma unroll
        for (int dt = 0; dt < 4; dt++) *(f32x4*)&d[2 + 4 * dt] = o[dt];
    }
    __syncthreads();
    if (ws == 0 && row < a.T) {
        float mm = m;
#pragma unroll
        for (int k = 1; k < NSET; k++) mm = fmaxf(mm, xch[18 * (256 * (k - 1) + ts)]);
        const float a0 = __builtin_amdgcn_exp2f(m - mm);
        float lt = l * a0;
        f32x4 ot[4];
#pragma unroll
        for (int dt = 0; dt < 4; dt++) ot[dt] = o[dt] * a0;
#pragma unroll
        for (int k = 1; k < NSET; k++) {
            const float* d = xch + 18 * (256 * (k - 1) + ts);
            const float a1 = d[0] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(d[0] - mm);
            lt = fmaf(d[1], a1, lt);
#pragma unroll
            for (int dt = 0; dt < 4; dt++) {
                const f32x4 o1 = *(const f32x4*)&d[2 + 4 * dt];
#pragma unroll
                for (int e = 0; e < 4; e++) ot[dt][e] = fmaf(o1[e], a1, ot[dt][e]);
            }
        }
        f32x4* op = (f32x4*)(a.out + ((int64_t)row * a.H + h) * DH + 16 * g);
#pragma unroll
        for (int e = 0; e < 4; e++) gst(op + e, f32x4{ot[0][e] / lt, ot[1][e] / lt, ot[2][e] / lt, ot[3][e] / lt});
    }
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

// head-group size: 2 KV heads when the count allows (a position's slice of
// the record is then >= 2 heads wide), else 1
inline int head_group(int Hkv) { return Hkv % 2 == 0 ? 2 : 1; }

size_t split_ws_bytes(int H, int nchunk) { return (size_t)nchunk * H * (2 + 64) * sizeof(float); }

template <int KF, int VF, int HG, bool FUSED>
int launch_split(SplitArgs a, int rep, size_t ws_bytes, void* ws, hipStream_t st) {
    constexpr int GS = 4 * (64 / (8 * HG));
    a.chunk = chunk_len(a.max_seq, GS);
    const int max_pos = a.d_pos ? a.max_seq : a.start_pos + 1;
    if constexpr (FUSED && KF == 0 && VF == 0) {
        // short fp32 caches: one launch, no partials (attn_vsplit_kernel)
        if (max_pos <= kVsMaxPos) {
            // one query head and 8 value dims per workgroup, as many steps
            // of 256 positions as the bound needs (measured at config 2's
            // shape, position 528, caches rotated past the MALL: 7.45 us
            // against 7.9 us for 8 lanes per position in 128-position steps
            // and 8.2 us for split + combine; 16 value slices per head
            // (512 workgroups) 11.1 us; 4 query heads x 16 dims per workgroup
            // with 8 lanes per position 10.2 us)
            const int nst = (max_pos + 255) / 256;
            const dim3 grid(a.H * 8);
            if (nst == 1) hipLaunchKernelGGL((attn_vsplit_kernel<8, 1>), grid, dim3(1024), 0, st, a);
            else if (nst == 2) hipLaunchKernelGGL((attn_vsplit_kernel<8, 2>), grid, dim3(1024), 0, st, a);
            else if (nst == 3) hipLaunchKernelGGL((attn_vsplit_kernel<8, 3>), grid, dim3(1024), 0, st, a);
            else hipLaunchKernelGGL((attn_vsplit_kernel<8, 4>), grid, dim3(1024), 0, st, a);
            return hipGetLastError() == hipSuccess ? RINA_OK : RINA_ERR_HIP;
        }
    }
    const int nchunk = (max_pos + a.chunk - 1) / a.chunk;
    if (!ws || ws_bytes < split_ws_bytes(a.H, nchunk)) return RINA_ERR_WORKSPACE;
    a.ws_m = (float*)ws;
    a.ws_l = a.ws_m + (size_t)nchunk * a.H;
    a.ws_o = a.ws_l + (size_t)nchunk * a.H;
    // x padded to a multiple of the 8 XCDs: workgroups are dealt to the XCDs
    // round-robin in linear order, so every head group of chunk c then runs
    // on the XCD of c and the cache lines that two groups' spans share are
    // fetched into one L2 (the padding workgroups start past max_seq and
    // return at once)
    dim3 grid((nchunk + 7) / 8 * 8, a.Hkv / HG);
    // an even head ratio splits a KV head's query heads over two wave sets
    // (512 threads): half the per-lane chain per position, two waves per SIMD
    switch (rep) {
        case 1: hipLaunchKernelGGL((attn_split_kernel<KF, VF, HG, 1, FUSED, 1>), grid, dim3(256), 0, st, a); break;
        case 2: hipLaunchKernelGGL((attn_split_kernel<KF, VF, HG, 2, FUSED, 2>), grid, dim3(512), 0, st, a); break;
        case 4: hipLaunchKernelGGL((attn_split_kernel<KF, VF, HG, 4, FUSED, 2>), grid, dim3(512), 0, st, a); break;
        case 8: hipLaunchKernelGGL((attn_split_kernel<KF, VF, HG, 8, FUSED, 2>), grid, dim3(512), 0, st, a); break;
        default: return RINA_ERR_SHAPE;
    }
    if (hipGetLastError() != hipSuccess) return RINA_ERR_HIP;
    hipLaunchKernelGGL(attn_combine_kernel, dim3(a.H), dim3(256), 0, st, a);
    return hipGetLastError() == hipSuccess ? RINA_OK : RINA_ERR_HIP;
}

template <int KF, int VF, bool FUSED>
int launch_split_hg(const SplitArgs& a, int rep, size_t ws_bytes, void* ws, hipStream_t st) {
    if (head_group(a.Hkv) == 2) return launch_split<KF, VF, 2, FUSED>(a, rep, ws_bytes, ws, st);
    return launch_split<KF, VF, 1, FUSED>(a, rep, ws_bytes, ws, st);
}

template <bool FUSED>
int launch_split_mode(const SplitArgs& a, int rep, size_t ws_bytes, void* ws, hipStream_t st) {
    switch (a.mode) {
        case RINA_KV_FP32: return launch_split_hg<0, 0, FUSED>(a, rep, ws_bytes, ws, st);
        case RINA_KV_Q8: return launch_split_hg<RINA_KVF_Q8_0, RINA_KVF_Q8_0, FUSED>(a, rep, ws_bytes, ws, st);
        case RINA_KV_Q4: return launch_split_hg<RINA_KVF_Q4_0, RINA_KVF_Q4_0, FUSED>(a, rep, ws_bytes, ws, st);
        case RINA_KV_Q4K_Q2V: return launch_split_hg<RINA_KVF_Q4_0, RINA_KVF_Q2_1, FUSED>(a, rep, ws_bytes, ws, st);
        case RINA_KV_Q2: return launch_split_hg<RINA_KVF_Q2_1, RINA_KVF_Q2_1, FUSED>(a, rep, ws_bytes, ws, st);
        default: return launch_split_hg<RINA_KVF_Q2_1, RINA_KVF_Q1_0, FUSED>(a, rep, ws_bytes, ws, st);
    }
}

bool rep_ok(int rep) { return rep == 1 || rep == 2 || rep == 4 || rep == 8; }

}  // namespace

extern "C" int rina_hip_gqa_one_launch_positions(void) { return kVsMaxPos; }

extern "C" size_t rina_hip_gqa_attention_workspace(int T, int H, int dh, int max_pos) {
    (void)T;
    (void)dh;
    if (H < 1 || max_pos < 1) return 0;
    // the smallest workgroup step (16 positions) gives the most chunks: an
    // upper bound for every head-group size
    const int cs = chunk_len(max_pos, 16);
    return split_ws_bytes(H, (max_pos + cs - 1) / cs);
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
    int rep = H / Hkv;
    bool fast = T == 1 && dh == 64 && !pre_rope && rep_ok(rep) && cache_k && cache_v &&
                ((uintptr_t)q % 16 == 0) && ((uintptr_t)kcur % 16 == 0) && ((uintptr_t)vcur % 16 == 0) &&
                (((uintptr_t)cache_k | (uintptr_t)cache_v) % (mode == RINA_KV_FP32 ? 16 : 2) == 0);
    if (fast) {   // (the split kernel's q8 windows assume 2-byte aligned records)
        SplitArgs sa{};
        sa.q = q; sa.kcur = kcur; sa.vcur = vcur;
        sa.ck = (uint8_t*)cache_k; sa.cv = (uint8_t*)cache_v;
        sa.out = out;
        sa.mode = mode; sa.H = H; sa.Hkv = Hkv; sa.start_pos = start_pos; sa.max_seq = max_seq; sa.d_pos = d_pos;
        sa.scale = 1.0f / sqrtf((float)dh);
        return launch_split_mode<false>(sa, rep, ws_bytes, workspace, st);
    }
    AttnArgs a{};
    a.q = q; a.kcur = kcur; a.vcur = vcur;
    a.ck = (const uint8_t*)cache_k; a.cv = (const uint8_t*)cache_v;
    a.rkc = rkc; a.rks = rks; a.out = out;
    a.mode = mode; a.pre_rope = pre_rope; a.T = T; a.H = H; a.Hkv = Hkv; a.dh = dh;
    a.start_pos = start_pos; a.max_seq = max_seq; a.d_pos = d_pos;
    a.scale = 1.0f / sqrtf((float)dh);
    // a prompt from position 0 reads only the current rows
    if (T > 1 && !d_pos && start_pos == 0 && dh == 64 && ((uintptr_t)kcur % 16 == 0)) {
        const int ntile = (T + kPromptRows - 1) / kPromptRows;
        if (rep % 4 == 0 && ((uintptr_t)q | (uintptr_t)vcur | (uintptr_t)out) % 16 == 0)
            hipLaunchKernelGGL(attn_prompt_mfma_kernel<2>, dim3(H / 4, ntile), dim3(512), 0, st, a);
        else
            hipLaunchKernelGGL(attn_prompt_kernel, dim3(H, ntile), dim3(64), 0, st, a);
        RINA_LAUNCH_CHECK();
        return RINA_OK;
    }
    hipLaunchKernelGGL(attn_generic_kernel, dim3(H, T), dim3(64), 0, st, a, kf, vf);
    RINA_LAUNCH_CHECK();
    return RINA_OK;
}

extern "C" int rina_hip_gqa_decode_attention(const float* q, const float* k, const float* v, const float* rope_q_cos,
                                             const float* rope_q_sin, const float* rope_k_cos,
                                             const float* rope_k_sin, void* cache_k, void* cache_v, int mode, int H,
                                             int Hkv, int dh, int start_pos, const int* d_pos, int max_seq,
                                             float* out, float* k_rot_out, void* workspace, size_t ws_bytes,
                                             void* stream) {
    if (!q || !k || !v || !out || !cache_k || !cache_v || H < 1 || Hkv < 1 || max_seq < 1) return RINA_ERR_ARG;
    if (mode < RINA_KV_FP32 || mode > RINA_KV_Q2K_Q1V) return RINA_ERR_QTYPE;
    if (H % Hkv || dh != 64 || !rep_ok(H / Hkv)) return RINA_ERR_SHAPE;
    if ((!rope_q_cos) != (!rope_q_sin) || (!rope_k_cos) != (!rope_k_sin)) return RINA_ERR_ARG;
    if (!d_pos && (start_pos < 0 || start_pos + 1 > max_seq)) return RINA_ERR_RANGE;
    const uintptr_t al = (uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)rope_q_cos | (uintptr_t)rope_q_sin |
                         (uintptr_t)rope_k_cos | (uintptr_t)rope_k_sin | (uintptr_t)k_rot_out;
    if (al % 16 || (mode == RINA_KV_FP32 && ((uintptr_t)cache_k | (uintptr_t)cache_v) % 16) ||
        (mode != RINA_KV_FP32 && ((uintptr_t)cache_k | (uintptr_t)cache_v) % 2))
        return RINA_ERR_SHAPE;
    SplitArgs sa{};
    sa.q = q; sa.kcur = k; sa.vcur = v;
    sa.qc = rope_q_cos; sa.qs = rope_q_sin; sa.kc = rope_k_cos; sa.ks = rope_k_sin;
    sa.ck = (uint8_t*)cache_k; sa.cv = (uint8_t*)cache_v; sa.k_rot_out = k_rot_out;
    sa.out = out;
    sa.mode = mode; sa.H = H; sa.Hkv = Hkv; sa.start_pos = start_pos; sa.max_seq = max_seq; sa.d_pos = d_pos;
    sa.scale = 1.0f / sqrtf((float)dh);
    return launch_split_mode<true>(sa, H / Hkv, ws_bytes, workspace, as_stream(stream));
}

// ---------------------------------------------------------------------------
// Allocation-free decode attention.  The chunk partials (m, l, O) that the
// caller's workspace holds for rina_hip_gqa_decode_attention live here in a
// file-scope device array instead: kNoAllocScratchBytes per device, held
// until the process ends.  Nothing in it has to start at zero (the combine
// reads only the chunks the split kernel of the same call wrote).  Host code
// never passes the array's name (a host-side stand-in); it looks up the
// array's device address once per device, with that device current, and
// passes that.  Every call on one device shares the array: calls that
// overlap on one device (two streams) race.
// ---------------------------------------------------------------------------
constexpr size_t kNoAllocScratchBytes = (size_t)1 << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {
void* g_scratch_addr[64];
std::mutex g_scratch_mu;

int noalloc_scratch(void** out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return RINA_ERR_HIP;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_addr[dev]) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return RINA_ERR_HIP;
        g_scratch_addr[dev] = p;
    }
    *out = g_scratch_addr[dev];
    return RINA_OK;
}
}  // namespace

extern "C" size_t rina_hip_noalloc_scratch_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int rina_hip_gqa_decode_attention_noalloc(const float* q, const float* k, const float* v,
                                                     const float* rope_q_cos, const float* rope_q_sin,
                                                     const float* rope_k_cos, const float* rope_k_sin, void* cache_k,
                                                     void* cache_v, int mode, int H, int Hkv, int dh, int start_pos,
                                                     const int* d_pos, int max_seq, float* out, float* k_rot_out,
                                                     void* stream) {
    if (H < 1 || max_seq < 1) return RINA_ERR_ARG;
    const size_t need = rina_hip_gqa_attention_workspace(1, H, dh, max_seq);
    if (need > kNoAllocScratchBytes) return RINA_ERR_WORKSPACE;
    void* ws = nullptr;
    const int rc = noalloc_scratch(&ws);
    if (rc) return rc;
    return rina_hip_gqa_decode_attention(q, k, v, rope_q_cos, rope_q_sin, rope_k_cos, rope_k_sin, cache_k, cache_v,
                                         mode, H, Hkv, dh, start_pos, d_pos, max_seq, out, k_rot_out, ws,
                                         kNoAllocScratchBytes, stream);
}

extern "C" size_t rina_hip_dq_attention_workspace(int H, int dq, int max_pos) {
    if (H < 1 || dq < 1 || max_pos < 1) return 0;
    (void)dq;
    const size_t nch = ((size_t)max_pos + kDqChunk - 1) / kDqChunk;
    return nch * H * (2 + 64) * sizeof(float);
}

namespace {
int dq_attention(const float* qa, const float* qb, const float* ka, const float* kb, const float* v,
                 const float* rope_q_cos, const float* rope_q_sin, const float* rope_k_cos, const float* rope_k_sin,
                 int kv_mode, float* cache_k, float* cache_v, uint8_t* cache_kc, float* cache_kr, uint8_t* cache_vq,
                 int H, int Hkv, int da, int db, int dv, int start_pos, const int* d_pos, int max_seq, float* out,
                 void* workspace, size_t ws_bytes, hipStream_t st) {
    if (!qa || !ka || !v || !out || H < 1 || Hkv < 1 || da < 1 || db < 0 || max_seq < 1) return RINA_ERR_ARG;
    if (db > 0 && (!qb || !kb)) return RINA_ERR_ARG;
    if (kv_mode == RINA_KV_FP32 && (!cache_k || !cache_v)) return RINA_ERR_ARG;
    if (kv_mode == RINA_KV_Q2K_Q1V && (!cache_kc || !cache_vq || (db > 0 && !cache_kr))) return RINA_ERR_ARG;
    if (kv_mode != RINA_KV_FP32 && kv_mode != RINA_KV_Q2K_Q1V) return RINA_ERR_QTYPE;
    if ((!rope_q_cos) != (!rope_q_sin) || (!rope_k_cos) != (!rope_k_sin)) return RINA_ERR_ARG;
    if (H % Hkv || dv != 64 || da + db > 128 || da + db < 64 || db % 2) return RINA_ERR_SHAPE;
    if (kv_mode == RINA_KV_Q2K_Q1V && (da != 64 || db > 64 || ((uintptr_t)cache_kc | (uintptr_t)cache_vq) % 2))
        return RINA_ERR_SHAPE;
    if (!d_pos && (start_pos < 0 || start_pos >= max_seq)) return RINA_ERR_RANGE;
    const int max_pos = d_pos ? max_seq : start_pos + 1;
    const int nch = (max_pos + kDqChunk - 1) / kDqChunk;
    if (nch > kMaxChunks) return RINA_ERR_SHAPE;                 // combine merges <= 64 chunks
    const size_t need = rina_hip_dq_attention_workspace(H, da + db, max_pos);
    if (!workspace || ws_bytes < need) return RINA_ERR_WORKSPACE;
    DqArgs a{};
    a.qa = qa; a.qb = qb; a.ka = ka; a.kb = kb; a.v = v;
    a.qc = rope_q_cos; a.qs = rope_q_sin; a.kc = rope_k_cos; a.ks = rope_k_sin;
    a.ck = cache_k; a.cv = cache_v; a.ckq = cache_kc; a.ckr = cache_kr; a.cvq = cache_vq;
    a.H = H; a.Hkv = Hkv; a.da = da; a.db = db; a.dv = dv;
    a.start_pos = start_pos; a.max_seq = max_seq; a.d_pos = d_pos;
    a.scale = 1.0f / sqrtf((float)(da + db));
    SplitArgs p{};
    p.ws_m = (float*)workspace;
    p.ws_l = p.ws_m + (size_t)nch * H;
    p.ws_o = p.ws_l + (size_t)nch * H;
    p.out = out; p.H = H; p.start_pos = start_pos; p.max_seq = max_seq; p.d_pos = d_pos; p.chunk = kDqChunk;
    // chunks padded to the 8 XCDs: the query heads of one chunk share its
    // cache rows in one L2 (padding workgroups start past max_seq and return)
    const dim3 grid((nch + 7) / 8 * 8, H);
    if (kv_mode == RINA_KV_FP32) hipLaunchKernelGGL(dq_split_kernel<0>, grid, dim3(256), 0, st, a, p);
    else hipLaunchKernelGGL(dq_split_kernel<1>, grid, dim3(256), 0, st, a, p);
    RINA_LAUNCH_CHECK();
    hipLaunchKernelGGL(attn_combine_kernel, dim3(H), dim3(256), 0, st, p);
    RINA_LAUNCH_CHECK();
    return RINA_OK;
}
}  // namespace

extern "C" int rina_hip_dq_decode_attention(const float* qa, const float* qb, const float* ka, const float* kb,
                                            const float* v, const float* rope_q_cos, const float* rope_q_sin,
                                            const float* rope_k_cos, const float* rope_k_sin, float* cache_k,
                                            float* cache_v, int H, int Hkv, int da, int db, int dv, int start_pos,
                                            const int* d_pos, int max_seq, float* out, void* workspace,
                                            size_t ws_bytes, void* stream) {
    return dq_attention(qa, qb, ka, kb, v, rope_q_cos, rope_q_sin, rope_k_cos, rope_k_sin, RINA_KV_FP32, cache_k,
                        cache_v, nullptr, nullptr, nullptr, H, Hkv, da, db, dv, start_pos, d_pos, max_seq, out,
                        workspace, ws_bytes, as_stream(stream));
}

extern "C" size_t rina_hip_dq_prompt_workspace(int T, int H, int Hkv, int da, int db, int dv) {
    if (T < 1 || H < 1 || Hkv < 1 || da < 1 || db < 0 || dv < 1) return 0;
    const size_t dq = (size_t)da + db, t = (size_t)T;
    return sizeof(float) * (2 * t * H * dq + 2 * t * Hkv * dq);
}

extern "C" int rina_hip_dq_prompt_attention(const float* qa, const float* qb, const float* ka, const float* kb,
                                            const float* v, const float* rope_q_cos, const float* rope_q_sin,
                                            const float* rope_k_cos, const float* rope_k_sin, float* cache_k,
                                            float* cache_v, int H, int Hkv, int da, int db, int dv, int T,
                                            int max_seq, float* out, void* workspace, size_t ws_bytes,
                                            void* stream) {
    if (!qa || !ka || !v || !cache_k || !cache_v || !out || H < 1 || Hkv < 1 || da < 1 || db < 0 || dv < 1 ||
        T < 1 || max_seq < 1 || (db > 0 && (!qb || !kb)) || db % 2)
        return RINA_ERR_ARG;
    if (H % Hkv || da + db > 256 || dv > da + db) return RINA_ERR_SHAPE;
    if (T > max_seq) return RINA_ERR_RANGE;
    const size_t need = rina_hip_dq_prompt_workspace(T, H, Hkv, da, db, dv);
    if (!workspace || ws_bytes < need || (uintptr_t)workspace % 16) return RINA_ERR_WORKSPACE;
    const int dq = da + db;
    float* q_full = (float*)workspace;
    float* o_full = q_full + (size_t)T * H * dq;
    float* k_full = o_full + (size_t)T * H * dq;
    float* v_full = k_full + (size_t)T * Hkv * dq;
    DqArgs a{};
    a.qa = qa; a.qb = qb; a.ka = ka; a.kb = kb; a.v = v;
    a.qc = rope_q_cos; a.qs = rope_q_sin; a.kc = rope_k_cos; a.ks = rope_k_sin;
    a.ck = cache_k; a.cv = cache_v;
    a.H = H; a.Hkv = Hkv; a.da = da; a.db = db; a.dv = dv; a.start_pos = 0; a.max_seq = max_seq;
    hipStream_t st = as_stream(stream);
    hipLaunchKernelGGL(dq_rows_kernel, dim3(T, H + Hkv), dim3(256), 0, st, a, q_full, k_full, v_full);
    RINA_LAUNCH_CHECK();
    // causal attention over the rows, scale 1/sqrt(da + db)
    int rc = rina_hip_gqa_attention(q_full, k_full, v_full, k_full, v_full, RINA_KV_FP32, 0, nullptr, nullptr, T, H,
                                    Hkv, dq, 0, nullptr, max_seq, o_full, nullptr, 0, stream);
    if (rc) return rc;
    if (hipMemcpy2DAsync(out, sizeof(float) * dv, o_full, sizeof(float) * dq, sizeof(float) * dv, (size_t)T * H,
                         hipMemcpyDeviceToDevice, st) != hipSuccess)
        return RINA_ERR_HIP;
    return RINA_OK;
}

extern "C" size_t rina_hip_dq_kv_region_bytes(int kv_mode, int part, int max_seq, int Hkv, int da, int db, int dv) {
    if (max_seq < 1 || Hkv < 1 || da < 1 || db < 0 || dv < 1 || part < 0 || part > 2) return 0;
    const size_t rows = (size_t)max_seq * Hkv;
    if (kv_mode == RINA_KV_FP32) return part == 0 ? rows * (da + db) * 4 : part == 1 ? rows * dv * 4 : 0;
    if (kv_mode != RINA_KV_Q2K_Q1V || da % 32 || dv % 32) return 0;
    return part == 0 ? rows * (da / 32) * 10 : part == 1 ? rows * (dv / 32) * 6 : rows * db * 4;
}

extern "C" int rina_hip_dq_decode_attention_kv(const float* qa, const float* qb, const float* ka, const float* kb,
                                               const float* v, const float* rope_q_cos, const float* rope_q_sin,
                                               const float* rope_k_cos, const float* rope_k_sin, int kv_mode,
                                               void* cache_k, void* cache_v, float* cache_kr, int H, int Hkv,
                                               int da, int db, int dv, int start_pos, const int* d_pos, int max_seq,
                                               float* out, void* workspace, size_t ws_bytes, void* stream) {
    if (kv_mode == RINA_KV_FP32)
        return dq_attention(qa, qb, ka, kb, v, rope_q_cos, rope_q_sin, rope_k_cos, rope_k_sin, kv_mode,
                            (float*)cache_k, (float*)cache_v, nullptr, nullptr, nullptr, H, Hkv, da, db, dv, start_pos,
                            d_pos, max_seq, out, workspace, ws_bytes, as_stream(stream));
    return dq_attention(qa, qb, ka, kb, v, rope_q_cos, rope_q_sin, rope_k_cos, rope_k_sin, kv_mode, nullptr, nullptr,
                        (uint8_t*)cache_k, cache_kr, (uint8_t*)cache_v, H, Hkv, da, db, dv, start_pos, d_pos, max_seq,
                        out, workspace, ws_bytes, as_stream(stream));
}

extern "C" int rina_hip_dq_prompt_attention_kv(const float* qa, const float* qb, const float* ka, const float* kb,
                                               const float* v, const float* rope_q_cos, const float* rope_q_sin,
                                               const float* rope_k_cos, const float* rope_k_sin, int kv_mode,
                                               void* cache_k, void* cache_v, float* cache_kr, int H, int Hkv,
                                               int da, int db, int dv, int start_pos, int T, int max_seq,
                                               float* out, void* stream) {
    if (!qa || !ka || !v || !out || H < 1 || Hkv < 1 || da < 1 || db < 0 || dv < 1 || T < 1 || max_seq < 1)
        return RINA_ERR_ARG;
    if (db > 0 && (!qb || !kb)) return RINA_ERR_ARG;
    if ((!rope_q_cos) != (!rope_q_sin) || (!rope_k_cos) != (!rope_k_sin)) return RINA_ERR_ARG;
    if (kv_mode != RINA_KV_FP32 && kv_mode != RINA_KV_Q2K_Q1V) return RINA_ERR_QTYPE;
    const bool packed = kv_mode == RINA_KV_Q2K_Q1V;
    if (!cache_k || !cache_v || (packed && db > 0 && !cache_kr)) return RINA_ERR_ARG;
    if (H % Hkv || dv != 64 || da + db > 128 || da + db < 64 || db % 2) return RINA_ERR_SHAPE;
    if (packed && (da != 64 || db > 64 || ((uintptr_t)cache_k | (uintptr_t)cache_v) % 2)) return RINA_ERR_SHAPE;
    if (!packed && ((uintptr_t)cache_k | (uintptr_t)cache_v) % 4) return RINA_ERR_SHAPE;
    if (start_pos < 0 || (int64_t)start_pos + T > max_seq) return RINA_ERR_RANGE;
    DqArgs a{};
    a.qa = qa; a.qb = qb; a.ka = ka; a.kb = kb; a.v = v;
    a.qc = rope_q_cos; a.qs = rope_q_sin; a.kc = rope_k_cos; a.ks = rope_k_sin;
    if (packed) { a.ckq = (uint8_t*)cache_k; a.ckr = cache_kr; a.cvq = (uint8_t*)cache_v; }
    else { a.ck = (float*)cache_k; a.cv = (float*)cache_v; }
    a.out = out;
    a.H = H; a.Hkv = Hkv; a.da = da; a.db = db; a.dv = dv; a.start_pos = start_pos; a.max_seq = max_seq;
    a.scale = 1.0f / sqrtf((float)(da + db));
    hipStream_t st = as_stream(stream);
    if (packed) hipLaunchKernelGGL(dq_pack_rows_kernel<1>, dim3(T, Hkv), dim3(64), 0, st, a);
    else hipLaunchKernelGGL(dq_pack_rows_kernel<0>, dim3(T, Hkv), dim3(64), 0, st, a);
    RINA_LAUNCH_CHECK();
    if (packed) hipLaunchKernelGGL(dq_prompt_kv_kernel<1>, dim3(T, H), dim3(256), 0, st, a);
    else hipLaunchKernelGGL(dq_prompt_kv_kernel<0>, dim3(T, H), dim3(256), 0, st, a);
    RINA_LAUNCH_CHECK();
    return RINA_OK;
}
