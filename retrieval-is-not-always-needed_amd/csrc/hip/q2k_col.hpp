// Q2_K / Q4 column helpers shared by the matvec and MoE kernels: block
// floating point activation digits, the 32-value Q2_K column dot, and the
// 4-byte aligned 16-byte loads of the 18/20/84-byte block formats.
#pragma once
#include "rina_common.hpp"

namespace {

enum { FMT_Q4_0 = 0, FMT_Q4_0F = 1, FMT_Q2_K = 2 };

typedef float f32x4 __attribute__((ext_vector_type(4)));

typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));

// 16-byte streaming load from a 4-byte aligned global address
__device__ __forceinline__ u32x4_a4 gld_nt_a4(const uint8_t* p) {
    return __builtin_nontemporal_load((const __attribute__((address_space(1))) u32x4_a4*)p);
}

// Activation columns owned by one lane, as block floating point: the column's
// values x_i = X_i * 2^(e-22) with integers |X_i| < 2^22 (e: exponent of the
// column's max |x|), and X_i split into three signed 8-bit digit planes
// X = d0 + 256 d1 + 65536 d2.  A weight block then needs only integer dot
// products (v_dot4c_i32_i8, 4 MACs per instruction, exact) and one fp32
// scale per block: the error is that of rounding x to 22 significant bits of
// its column maximum, below the fp32 accumulation error of the reference loop.
// Plane dword t of a Q4 column holds the digits of values 8(t/2)+2b+(t%2),
// b = 0..3: the order of the nibble bytes after the low/high split.
// Digits of four values at once.  With Y = X + 0x808080 (|X| < 2^22, so
// 0 <= Y < 2^24), byte k of Y minus 128 is digit d_k of the centered
// base-256 split X = d0 + 256 d1 + 65536 d2 (d_k in [-128, 127]), and as an
// int8 bit pattern y_k - 128 is y_k ^ 0x80: the digit bytes are the bytes of
// Y ^ 0x808080.  v_perm_b32 then gathers byte k of the four values into
// plane dword k.
__device__ __forceinline__ uint32_t zdig(float v, float up) {
    return (uint32_t)((int)rintf(v * up) + 0x808080) ^ 0x808080u;
}

__device__ __forceinline__ void digits4(float v0, float v1, float v2, float v3, float up, uint32_t& p0,
                                        uint32_t& p1, uint32_t& p2) {
    const uint32_t z0 = zdig(v0, up), z1 = zdig(v1, up), z2 = zdig(v2, up), z3 = zdig(v3, up);
    const uint32_t t01 = __builtin_amdgcn_perm(z1, z0, 0x05010400u);   // z0.b0 z1.b0 z0.b1 z1.b1
    const uint32_t t23 = __builtin_amdgcn_perm(z3, z2, 0x05010400u);
    const uint32_t u01 = __builtin_amdgcn_perm(z1, z0, 0x00000602u);   // z0.b2 z1.b2 . .
    const uint32_t u23 = __builtin_amdgcn_perm(z3, z2, 0x00000602u);
    p0 = __builtin_amdgcn_perm(t23, t01, 0x05040100u);
    p1 = __builtin_amdgcn_perm(t23, t01, 0x07060302u);
    p2 = __builtin_amdgcn_perm(u23, u01, 0x05040100u);
}

// sum of the four signed digit bytes of a plane dword
__device__ __forceinline__ int dsum4(uint32_t p, int acc) {
    return __builtin_amdgcn_sdot4((int)p, 0x01010101, acc, false);
}

template <int FMT, int CPL>
struct XCols {
    static constexpr int UNIT = (FMT == FMT_Q2_K) ? 16 : 32;
    static constexpr int ND = UNIT / 4;   // dwords per digit plane
    int32_t dg[CPL][3][ND];
    float tt[CPL][3];   // 7 * (sum of plane digits): the -7 nibble offset
    float xe[CPL];      // 2^(e-22)
    float xs[CPL];      // fp32 sum of the column (Q2_K min term)
};

template <int FMT, int CPL>
__device__ __forceinline__ void digitize(XCols<FMT, CPL>& xc, int j, const float (&x)[XCols<FMT, CPL>::UNIT]) {
    constexpr int UNIT = XCols<FMT, CPL>::UNIT;
    float mx = 0.f, sum = 0.f;
#pragma unroll
    for (int i = 0; i < UNIT; i++) { mx = fmaxf(mx, fabsf(x[i])); sum += x[i]; }
    int e = 0;
    if (mx > 0.f) (void)frexpf(mx, &e);            // mx < 2^e
    const float up = ldexpf(1.0f, 22 - e);
    xc.xe[j] = ldexpf(1.0f, e - 22);
    xc.xs[j] = sum;
    int s0 = 0, s1 = 0, s2 = 0;
#pragma unroll
    for (int t = 0; t < XCols<FMT, CPL>::ND; t++) {
        auto kk = [&](int b) { return (FMT == FMT_Q2_K) ? 4 * t + b : 8 * (t >> 1) + 2 * b + (t & 1); };
        uint32_t p0, p1, p2;
        digits4(x[kk(0)], x[kk(1)], x[kk(2)], x[kk(3)], up, p0, p1, p2);
        s0 = dsum4(p0, s0); s1 = dsum4(p1, s1); s2 = dsum4(p2, s2);
        xc.dg[j][0][t] = (int32_t)p0;
        xc.dg[j][1][t] = (int32_t)p1;
        xc.dg[j][2][t] = (int32_t)p2;
    }
    xc.tt[j][0] = 7.0f * (float)s0;
    xc.tt[j][1] = 7.0f * (float)s1;
    xc.tt[j][2] = 7.0f * (float)s2;
}

__device__ __forceinline__ float silu_mul(float g, float u) { return (g / (1.0f + expf(-g))) * u; }

// Column registers of the direct kernel: 32 values (8 dwords per plane) for
// every format.
template <int FMT>
using DCols = XCols<FMT == FMT_Q2_K ? FMT_Q4_0 : FMT, 1>;

__device__ __forceinline__ uint32_t funnel(uint32_t lo, uint32_t hi, uint32_t sh) {
    return (uint32_t)((((uint64_t)hi << 32) | lo) >> sh);
}

// exact integer sum_i (q_i - 7) X_i of one Q4 block (nib: its 16 nibble bytes), as float
template <int FMT, int CPL>
__device__ __forceinline__ float q4_dot(const uint32_t (&nib)[4], const XCols<FMT, CPL>& xc, int j) {
    int a0 = 0, a1 = 0, a2 = 0;
#pragma unroll
    for (int d = 0; d < 4; d++) {
        const int lo = (int)and_opaque(nib[d], 0x0F0F0F0Fu), hi = (int)and_opaque(nib[d] >> 4, 0x0F0F0F0Fu);
        a0 = __builtin_amdgcn_sdot4(lo, xc.dg[j][0][2 * d], a0, false);
        a1 = __builtin_amdgcn_sdot4(lo, xc.dg[j][1][2 * d], a1, false);
        a2 = __builtin_amdgcn_sdot4(lo, xc.dg[j][2][2 * d], a2, false);
        a0 = __builtin_amdgcn_sdot4(hi, xc.dg[j][0][2 * d + 1], a0, false);
        a1 = __builtin_amdgcn_sdot4(hi, xc.dg[j][1][2 * d + 1], a1, false);
        a2 = __builtin_amdgcn_sdot4(hi, xc.dg[j][2][2 * d + 1], a2, false);
    }
    const float f0 = (float)a0 - xc.tt[j][0], f1 = (float)a1 - xc.tt[j][1], f2 = (float)a2 - xc.tt[j][2];
    return fmaf(65536.0f, f2, fmaf(256.0f, f1, f0));
}

// One Q4 block (18-byte Q4_0 with fp16 scale, 20-byte Q4_0F with fp32 scale)
// at p: its scale and 16 nibble bytes, 4-byte aligned loads.
template <int FMT>
__device__ __forceinline__ void load_q4_block(const uint8_t* p, float& sc, uint32_t (&nib)[4]) {
    if constexpr (FMT == FMT_Q4_0F) {
        const u32x4_a4 v = gld_nt_a4(p);
        const uint32_t t = gld_nt((const uint32_t*)(p + 16));
        sc = __uint_as_float(v.x);
        nib[0] = v.y; nib[1] = v.z; nib[2] = v.w; nib[3] = t;
    } else {
        // 18-byte block: 20-byte window from the dword at or below its start
        const uintptr_t al = (uintptr_t)p & ~(uintptr_t)3;
        const uint32_t sh = (uint32_t)((uintptr_t)p & 3) * 8;        // 0 or 16
        const u32x4_a4 v = gld_nt_a4((const uint8_t*)al);
        const uint32_t t = gld_nt((const uint32_t*)(al + 16));
        const uint32_t d[5] = {v.x, v.y, v.z, v.w, t};
        sc = f16_to_f32(sh ? (d[0] >> 16) : (d[0] & 0xFFFF));
#pragma unroll
        for (int k = 0; k < 4; k++) nib[k] = (uint32_t)((((uint64_t)d[k + 1] << 32) | d[k]) >> (16 + sh));
    }
}

// One 32-value Q2_K column: exact integer dots of the two 16-value halves
// (shift sh selects the lane's 2-bit field of each qs byte), weighted by the
// halves' 4-bit scales, then d * 2^(e-22) * sum - dmin * (m0 x0 + m1 x1)
// with x0, x1 the fp32 half sums.
__device__ __forceinline__ float q2_col(const uint32_t (&qs)[8], uint32_t sm, uint32_t dd, int sh,
                                        const DCols<FMT_Q2_K>& xc) {
    int p0[3] = {0, 0, 0}, p1[3] = {0, 0, 0};
#pragma unroll
    for (int d = 0; d < 4; d++) {
        const int t0 = (int)and_opaque(qs[d] >> sh, 0x03030303u);
        const int t1 = (int)and_opaque(qs[4 + d] >> sh, 0x03030303u);
#pragma unroll
        for (int k = 0; k < 3; k++) {
            p0[k] = __builtin_amdgcn_sdot4(t0, xc.dg[0][k][d], p0[k], false);
            p1[k] = __builtin_amdgcn_sdot4(t1, xc.dg[0][k][4 + d], p1[k], false);
        }
    }
    // |p| <= 16 * 3 * 128: the scale products fit the 24-bit multiplier
    const int sc0 = (int)(sm & 0xF), sc1 = (int)((sm >> 8) & 0xF);
    const float f0 = (float)(__mul24(sc0, p0[0]) + __mul24(sc1, p1[0]));
    const float f1 = (float)(__mul24(sc0, p0[1]) + __mul24(sc1, p1[1]));
    const float f2 = (float)(__mul24(sc0, p0[2]) + __mul24(sc1, p1[2]));
    const float f = fmaf(65536.0f, f2, fmaf(256.0f, f1, f0));
    const float mn = fmaf((float)((sm >> 12) & 0xF), xc.tt[0][1], (float)((sm >> 4) & 0xF) * xc.tt[0][0]);
    return fmaf(f16_to_f32(dd & 0xFFFF) * xc.xe[0], f, -(f16_to_f32(dd >> 16) * mn));
}

// The loads of one 32-value Q2_K column starting at flat element e0 of the
// weight stream w (e0 % 32 == 0): the page's qs bytes, the two half scale
// bytes and the block's d / dmin.  The fields hold loaded dwords as they
// are (the field shift sh comes from the address; the scale pair is cut
// out of its dword where it is used): arithmetic on a loaded value at issue,
// also the zero extension of a 16-bit load, makes the wave wait for that
// load there.
struct Q2Col {
    uint32_t qs[8];
    uint32_t sm;    // dword holding the two half scale bytes (q2_sm16)
    uint32_t dd;
    uint32_t sh;    // 2g: shift of the column's 2-bit field in each qs byte
};

// the column's half scale bytes from the dword at 8 page + 4 (g / 2)
__device__ __forceinline__ uint32_t q2_sm16(uint32_t smw, uint32_t sh) { return smw >> (8 * (sh & 2)); }

__device__ __forceinline__ void q2_col_load(const uint8_t* bp, int page, int g, Q2Col& c) {
    const u32x4_a4 q0 = gld_nt_a4(bp + 16 + 32 * page), q1 = gld_nt_a4(bp + 32 + 32 * page);
    c.qs[0] = q0.x; c.qs[1] = q0.y; c.qs[2] = q0.z; c.qs[3] = q0.w;
    c.qs[4] = q1.x; c.qs[5] = q1.y; c.qs[6] = q1.z; c.qs[7] = q1.w;
    c.sm = gld_nt((const uint32_t*)(bp + 8 * page + 4 * (g >> 1)));
    c.dd = gld_nt((const uint32_t*)(bp + 80));
    c.sh = (uint32_t)(2 * g);
}

__device__ __forceinline__ void q2_col_issue(const uint8_t* w, int64_t e0, Q2Col& c) {
    const uint8_t* bp = w + (e0 >> 8) * 84;
    const int page = (int)(e0 >> 7) & 1, g = (int)(e0 >> 5) & 3;
    q2_col_load(bp, page, g, c);
}

// Same for a column inside one matrix of fewer than 2^32 values: 32-bit
// offset arithmetic.
__device__ __forceinline__ void q2_col_issue32(const uint8_t* w, uint32_t e0, Q2Col& c) {
    q2_col_load(w + (e0 >> 8) * 84u, (int)(e0 >> 7) & 1, (int)(e0 >> 5) & 3, c);
}

__device__ __forceinline__ float q2_col(const Q2Col& c, const DCols<FMT_Q2_K>& xc) {
    return q2_col(c.qs, q2_sm16(c.sm, c.sh), c.dd, (int)c.sh, xc);
}

// Quad form of the column loads.  When lane u holds column u of a row
// (e0 = row K + 32u, K % 128 == 0), the four lanes of a quad hold the
// columns g = 0..3 of one half page, and their 2-bit fields live in the same
// 32 qs bytes.  Each lane loads one quarter (8 bytes) and the quarters are
// exchanged with DPP quad broadcasts where the column is used, so the qs
// bytes pass through the load path once instead of four times.  All four
// lanes of a quad must be active at the exchange.
struct Q2ColQ {
    uint32_t q[2];  // qs bytes 8t .. 8t + 7 of the half page, t = lane & 3
    uint32_t sm;    // as Q2Col
    uint32_t dd;
    uint32_t sh;
};

__device__ __forceinline__ void q2_colq_load(const uint8_t* bp, int page, int g, Q2ColQ& c) {
    typedef uint32_t u32x2_a4 __attribute__((ext_vector_type(2), aligned(4)));
    const u32x2_a4 q = __builtin_nontemporal_load(
        (const __attribute__((address_space(1))) u32x2_a4*)(bp + 16 + 32 * page + 8 * (threadIdx.x & 3)));
    c.q[0] = q.x; c.q[1] = q.y;
    c.sm = gld_nt((const uint32_t*)(bp + 8 * page + 4 * (g >> 1)));
    c.dd = gld_nt((const uint32_t*)(bp + 80));
    c.sh = (uint32_t)(2 * g);
}

__device__ __forceinline__ void q2_colq_issue32(const uint8_t* w, uint32_t e0, Q2ColQ& c) {
    q2_colq_load(w + (e0 >> 8) * 84u, (int)(e0 >> 7) & 1, (int)(e0 >> 5) & 3, c);
}

__device__ __forceinline__ void q2_colq_issue(const uint8_t* w, int64_t e0, Q2ColQ& c) {
    q2_colq_load(w + (e0 >> 8) * 84, (int)(e0 >> 7) & 1, (int)(e0 >> 5) & 3, c);
}

// value of lane K of the quad in every lane of the quad: ds_swizzle in
// quad-permute mode (bit 15 set, lane selects in bits 0-7), which runs on the
// LDS crossbar instead of the vector ALU these kernels are bound by
template <int K>
__device__ __forceinline__ uint32_t quad_bcast(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, 0x8000 | (K * 0x55));
}

__device__ __forceinline__ void q2_colq_expand(const Q2ColQ& c, Q2Col& o) {
    o.qs[0] = quad_bcast<0>(c.q[0]); o.qs[1] = quad_bcast<0>(c.q[1]);
    o.qs[2] = quad_bcast<1>(c.q[0]); o.qs[3] = quad_bcast<1>(c.q[1]);
    o.qs[4] = quad_bcast<2>(c.q[0]); o.qs[5] = quad_bcast<2>(c.q[1]);
    o.qs[6] = quad_bcast<3>(c.q[0]); o.qs[7] = quad_bcast<3>(c.q[1]);
    o.sm = c.sm;
    o.dd = c.dd;
    o.sh = c.sh;
}

// Digits of one 32-value column in the Q2_K (natural) order with the fp32
// sums of its two halves, as the matvec kernels' workgroup prep makes them.
__device__ __forceinline__ void digitize_q2col(DCols<FMT_Q2_K>& xc, const float (&x)[32]) {
    float mx = 0.f, h0 = 0.f, h1 = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i++) {
        mx = fmaxf(mx, fabsf(x[i]));
        if (i < 16) h0 += x[i];
        else h1 += x[i];
    }
    int e = 0;
    if (mx > 0.f) (void)frexpf(mx, &e);            // mx < 2^e
    const float up = ldexpf(1.0f, 22 - e);
#pragma unroll
    for (int t = 0; t < 8; t++) {
        uint32_t p0, p1, p2;
        digits4(x[4 * t], x[4 * t + 1], x[4 * t + 2], x[4 * t + 3], up, p0, p1, p2);
        xc.dg[0][0][t] = (int32_t)p0;
        xc.dg[0][1][t] = (int32_t)p1;
        xc.dg[0][2][t] = (int32_t)p2;
    }
    xc.tt[0][0] = h0;
    xc.tt[0][1] = h1;
    xc.tt[0][2] = 0.f;
    xc.xe[0] = ldexpf(1.0f, e - 22);
    xc.xs[0] = 0.f;
}

// Activation source of the workgroup prep: x [K] and the optional norm
// prologue's weight and epsilon.
struct PrepSrc {
    const float* x;
    const float* nw;
    int K;
    float eps;
    float* xn = nullptr;   // with a norm prologue: workgroup 0 stores the normalized row here
};

// Workgroup-cooperative activation prep for the direct kernel: the K values
// are split over the 256 threads (TPC threads per 32-value column, 8..32
// values each) instead of every wave digitizing the whole row; the optional
// norm prologue reduces over the workgroup.  Digit planes, offsets and
// exponents go to LDS as [plane][dword][column] so each consumer lane then
// reads its column conflict-free.
struct PrepLds {
    int32_t dg[3][8][256];
    float tt[3][256];
    float xe[256];
    float red[8];
};

__device__ __forceinline__ float block_sum4(float v, float* red, int slot) {
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) red[slot * 4 + (threadIdx.x >> 6)] = v;
    __syncthreads();
    return (red[slot * 4 + 0] + red[slot * 4 + 1]) + (red[slot * 4 + 2] + red[slot * 4 + 3]);
}

// sum / max over groups of TPC consecutive lanes (TPC 1, 2 or 4)
template <int TPC>
__device__ __forceinline__ float grp_max(float v) {
    if (TPC >= 2) v = fmaxf(v, dpp_f<0xB1>(v));
    if (TPC >= 4) v = fmaxf(v, dpp_f<0x4E>(v));
    return v;
}
template <int TPC>
__device__ __forceinline__ int grp_sum_i(int v) {
    if (TPC >= 2) v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xf, 0xf, false);
    if (TPC >= 4) v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xf, 0xf, false);
    return v;
}
template <int TPC>
__device__ __forceinline__ float grp_sum_f(float v) {
    if (TPC >= 2) v += dpp_f<0xB1>(v);
    if (TPC >= 4) v += dpp_f<0x4E>(v);
    return v;
}

template <int TPC, int PRO>
struct PrepRaw {
    static constexpr int VPC = 32 / TPC;           // values per thread
    float x[VPC];
    float w[PRO != RINA_PRO_NONE ? VPC : 1];
};

// issued before the weight loads: vmcnt retires loads in issue order
template <int TPC, int PRO>
__device__ __forceinline__ void wg_prep_load(const PrepSrc& a, PrepRaw<TPC, PRO>& r) {
    constexpr int VPC = 32 / TPC;
    const int tid = threadIdx.x;
    const int u = tid / TPC, j = tid % TPC;
    const bool on = u < a.K / 32;
    float (&x)[VPC] = r.x;
    auto& w = r.w;
    {
        const int uu = on ? u : 0;
        const f32x4* xp = (const f32x4*)(a.x + (int64_t)uu * 32 + j * VPC);
#pragma unroll
        for (int i = 0; i < VPC / 4; i++) {
            f32x4 v = gld(xp + i);
            x[4 * i] = v.x; x[4 * i + 1] = v.y; x[4 * i + 2] = v.z; x[4 * i + 3] = v.w;
        }
        if constexpr (PRO != RINA_PRO_NONE) {
            const f32x4* wp = (const f32x4*)(a.nw + (int64_t)uu * 32 + j * VPC);
#pragma unroll
            for (int i = 0; i < VPC / 4; i++) {
                f32x4 v = gld(wp + i);
                w[4 * i] = v.x; w[4 * i + 1] = v.y; w[4 * i + 2] = v.z; w[4 * i + 3] = v.w;
            }
        }
    }
}

// Q4 columns: digit dword t holds the nibble order 8(t/2) + 2b + (t%2); tt =
// 7 * plane digit sums (the -7 offset).  Q2_K columns: natural order 4t + b;
// tt[0], tt[1] = fp32 sums of the two 16-value halves (the dmin * m term).
template <int FMT, int TPC, int PRO>
__device__ __forceinline__ void wg_prep_x(const PrepSrc& a, PrepRaw<TPC, PRO>& r, PrepLds& L) {
    constexpr int VPC = 32 / TPC;
    const int tid = threadIdx.x;
    const int u = tid / TPC, j = tid % TPC;
    const bool on = u < a.K / 32;
    float (&x)[VPC] = r.x;
    auto& w = r.w;
    if (!on) {
#pragma unroll
        for (int i = 0; i < VPC; i++) x[i] = 0.f;
    }
    if constexpr (PRO != RINA_PRO_NONE) {
        const float d = (float)a.K;
        float mean = 0.f;
        if (PRO == RINA_PRO_LAYERNORM) {
            float sm = 0.f;
#pragma unroll
            for (int i = 0; i < VPC; i++) sm += x[i];
            mean = block_sum4(sm, L.red, 0) / d;
        }
        float ss = 0.f;
        if (on) {
#pragma unroll
            for (int i = 0; i < VPC; i++) {
                const float t = x[i] - mean;
                ss = fmaf(t, t, ss);
            }
        }
        const float inv = 1.0f / sqrtf(block_sum4(ss, L.red, 1) / d + a.eps);
#pragma unroll
        for (int i = 0; i < VPC; i++) x[i] = on ? (x[i] - mean) * inv * w[i] : 0.f;
        if (a.xn && blockIdx.x == 0 && on) {
            f32x4* xo = (f32x4*)(a.xn + (int64_t)u * 32 + j * VPC);
#pragma unroll
            for (int i = 0; i < VPC / 4; i++) gst(xo + i, f32x4{x[4 * i], x[4 * i + 1], x[4 * i + 2], x[4 * i + 3]});
        }
    }
    float mx = 0.f;
#pragma unroll
    for (int i = 0; i < VPC; i++) mx = fmaxf(mx, fabsf(x[i]));
    mx = grp_max<TPC>(mx);
    int e = 0;
    if (mx > 0.f) (void)frexpf(mx, &e);            // mx < 2^e
    const float up = ldexpf(1.0f, 22 - e);
    int s0 = 0, s1 = 0, s2 = 0;
#pragma unroll
    for (int tl = 0; tl < VPC / 4; tl++) {         // local dword pair index tl/2, parity tl%2
        auto kk = [&](int b) { return FMT == FMT_Q2_K ? 4 * tl + b : 8 * (tl >> 1) + 2 * b + (tl & 1); };
        uint32_t p0, p1, p2;
        digits4(x[kk(0)], x[kk(1)], x[kk(2)], x[kk(3)], up, p0, p1, p2);
        if constexpr (FMT != FMT_Q2_K) { s0 = dsum4(p0, s0); s1 = dsum4(p1, s1); s2 = dsum4(p2, s2); }
        if (on) {
            const int t = j * (VPC / 4) + tl;
            L.dg[0][t][u] = (int32_t)p0;
            L.dg[1][t][u] = (int32_t)p1;
            L.dg[2][t][u] = (int32_t)p2;
        }
    }
    if constexpr (FMT == FMT_Q2_K) {
        float h0 = 0.f, h1 = 0.f;
#pragma unroll
        for (int i = 0; i < VPC; i++) {
            if (j * VPC + i < 16) h0 += x[i];
            else h1 += x[i];
        }
        h0 = grp_sum_f<TPC>(h0);
        h1 = grp_sum_f<TPC>(h1);
        if (on && j == 0) {
            L.tt[0][u] = h0;
            L.tt[1][u] = h1;
            L.tt[2][u] = 0.f;
            L.xe[u] = ldexpf(1.0f, e - 22);
        }
    } else {
        s0 = grp_sum_i<TPC>(s0);
        s1 = grp_sum_i<TPC>(s1);
        s2 = grp_sum_i<TPC>(s2);
        if (on && j == 0) {
            L.tt[0][u] = 7.0f * (float)s0;
            L.tt[1][u] = 7.0f * (float)s1;
            L.tt[2][u] = 7.0f * (float)s2;
            L.xe[u] = ldexpf(1.0f, e - 22);
        }
    }
    __syncthreads();
}

// Prep for four waves per row (K > 4096): thread t prepares column t, which
// is the column lane t % 64 of wave t / 64 consumes, so the digits go
// straight to the thread's registers (the same digits as the LDS path, bit
// for bit) with no LDS exchange, and without a norm prologue no barrier.
template <int FMT, int PRO>
__device__ __forceinline__ void own_prep_x(const PrepSrc& a, PrepRaw<1, PRO>& r, float* red, DCols<FMT>& xc) {
    const int u = threadIdx.x;
    const bool on = u < a.K / 32;
    float (&x)[32] = r.x;
    if (!on) {
#pragma unroll
        for (int i = 0; i < 32; i++) x[i] = 0.f;
    }
    if constexpr (PRO != RINA_PRO_NONE) {
        const float d = (float)a.K;
        float mean = 0.f;
        if (PRO == RINA_PRO_LAYERNORM) {
            float sm = 0.f;
#pragma unroll
            for (int i = 0; i < 32; i++) sm += x[i];
            mean = block_sum4(sm, red, 0) / d;
        }
        float ss = 0.f;
        if (on) {
#pragma unroll
            for (int i = 0; i < 32; i++) {
                const float t = x[i] - mean;
                ss = fmaf(t, t, ss);
            }
        }
        const float inv = 1.0f / sqrtf(block_sum4(ss, red, 1) / d + a.eps);
#pragma unroll
        for (int i = 0; i < 32; i++) x[i] = on ? (x[i] - mean) * inv * r.w[i] : 0.f;
        if (a.xn && blockIdx.x == 0 && on) {
            f32x4* xo = (f32x4*)(a.xn + (int64_t)u * 32);
#pragma unroll
            for (int i = 0; i < 8; i++) gst(xo + i, f32x4{x[4 * i], x[4 * i + 1], x[4 * i + 2], x[4 * i + 3]});
        }
    }
    if constexpr (FMT == FMT_Q2_K) digitize_q2col(xc, x);
    else digitize<FMT, 1>(xc, 0, x);
}

template <int FMT>
__device__ __forceinline__ void read_cols(const PrepLds& L, int u, bool active, DCols<FMT>& xc) {
    const int uu = active ? u : 0;
#pragma unroll
    for (int p = 0; p < 3; p++) {
#pragma unroll
        for (int t = 0; t < 8; t++) xc.dg[0][p][t] = L.dg[p][t][uu];
        xc.tt[0][p] = L.tt[p][uu];
    }
    xc.xe[0] = L.xe[uu];
    xc.xs[0] = 0.f;
}

}  // namespace
