// Shared device helpers for the gfx950 kernels of the RINA decode hot path.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "rina_hip.h"

#define RINA_WAVE 64

// ---------------------------------------------------------------------------
// fp16 <-> fp32
// ---------------------------------------------------------------------------

// fp32 -> fp16 bits, IEEE round-to-nearest-even, subnormals kept, overflow to
// inf (the semantics of __float2half that the reference KV quantizers use,
// kernels/quantize.cu:89,148,204,263).  Integer-only so the result does not
// depend on the MODE register's rounding/denormal state.
__device__ __forceinline__ uint32_t f32_to_f16_rne(float f) {
    uint32_t x = __float_as_uint(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u)
        return sign | (ax > 0x7f800000u ? (0x7e00u | ((ax >> 13) & 0x3ffu)) : 0x7c00u);
    if (ax >= 0x38800000u) {                       // |f| >= 2^-14: normal f16 range
        if (ax >= 0x47800000u) return sign | 0x7c00u;   // exponent > 15
        uint32_t h = ((ax >> 13) - (112u << 10));       // rebias 127 -> 15
        uint32_t rem = ax & 0x1fffu;
        h += (rem > 0x1000u) | ((rem == 0x1000u) & (h & 1u));
        return sign | h;                                // carry may give inf: correct
    }
    if (ax < 0x33000000u) return sign;             // < 2^-25: rounds to zero
    uint32_t e = ax >> 23;                         // 102..112
    uint32_t m = (ax & 0x7fffffu) | 0x800000u;
    uint32_t s = 126u - e;                         // 14..24
    uint32_t r = m >> s;
    uint32_t rem = m & ((1u << s) - 1u);
    uint32_t half = 1u << (s - 1u);
    r += (rem > half) | ((rem == half) & (r & 1u));
    return sign | r;
}

// fp16 bits -> fp32 (exact).
__device__ __forceinline__ float f16_to_f32(uint32_t h) {
    _Float16 v;
    uint16_t b = (uint16_t)h;
    __builtin_memcpy(&v, &b, 2);
    return (float)v;
}

// ---------------------------------------------------------------------------
// global-memory loads
// ---------------------------------------------------------------------------
// Pointers that reach a kernel inside an argument struct are generic; loads
// through them become FLAT instructions, which also count in LGKM_CNT, so any
// later LDS access waits for every outstanding weight prefetch.  These
// helpers cast to the global address space so the loads stay GLOBAL_LOAD.
template <typename T>
__device__ __forceinline__ T gld(const T* p) {
    return *(const __attribute__((address_space(1))) T*)p;
}
template <typename T>
__device__ __forceinline__ T gld_nt(const T* p) {   // streaming (non-temporal) load
    return __builtin_nontemporal_load((const __attribute__((address_space(1))) T*)p);
}
template <typename T>
__device__ __forceinline__ void gst(T* p, T v) {
    *(__attribute__((address_space(1))) T*)p = v;
}

// v_and_b32 the compiler cannot fold into per-field extracts, so the four
// bytes of the result feed v_cvt_f32_ubyte0..3 directly.
__device__ __forceinline__ uint32_t and_opaque(uint32_t a, uint32_t m) {
    uint32_t r;
    asm("v_and_b32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(m));
    return r;
}

// ---------------------------------------------------------------------------
// wave64 reductions through DPP (no LDS)
// ---------------------------------------------------------------------------

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Sum over each group of 8 consecutive lanes, result in every lane of the group.
__device__ __forceinline__ float sum8(float v) {
    v += dpp_f<0xB1>(v);    // quad_perm [1,0,3,2]
    v += dpp_f<0x4E>(v);    // quad_perm [2,3,0,1]
    v += dpp_f<0x141>(v);   // row_half_mirror
    return v;
}

// Sum over each DPP row (16 lanes), result in every lane of the row.
__device__ __forceinline__ float sum16(float v) {
    v = sum8(v);
    v += dpp_f<0x140>(v);   // row_mirror
    return v;
}

// DPP with a row mask: rows outside ROWS read 0 (the identity of the adds below).
template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_rows(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWS, 0xf, false));
}

// Sum over the whole wave, result uniform.  After the row sums R0..R3,
// row_bcast:15 adds R0 into row 1 and R2 into row 3, row_bcast:31 adds row
// 1's (R1 + R0) into row 3, and lane 63 holds (R3 + R2) + (R1 + R0): the
// pairing (R0 + R1) + (R2 + R3), bit for bit, with one readlane.
__device__ __forceinline__ float wave_sum(float v) {
    v = sum16(v);
    v += dpp_rows<0x142, 0xA>(v);   // row_bcast:15 into rows 1, 3
    v += dpp_rows<0x143, 0xC>(v);   // row_bcast:31 into rows 2, 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    v = fmaxf(v, dpp_f<0x140>(v));
    float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// Copy n floats from global memory to LDS with the whole workgroup, 16-byte
// loads when both ends allow, unrolled so the loads of several iterations
// are in flight together (a plain strided loop issues one load per round
// trip).
__device__ __forceinline__ void stage_lds(float* dst, const float* src, int n) {
    typedef float f32x4_s __attribute__((ext_vector_type(4)));
    const int tid = threadIdx.x, nt = blockDim.x;
    if (((uintptr_t)src % 16) == 0 && ((uintptr_t)dst % 16) == 0) {
        const int n4 = n >> 2;
        const f32x4_s* s4 = (const f32x4_s*)src;
        f32x4_s* d4 = (f32x4_s*)dst;
#pragma unroll 4
        for (int i = tid; i < n4; i += nt) d4[i] = gld(s4 + i);
        for (int i = 4 * n4 + tid; i < n; i += nt) dst[i] = gld(src + i);
    } else {
#pragma unroll 8
        for (int i = tid; i < n; i += nt) dst[i] = gld(src + i);
    }
}

// ---------------------------------------------------------------------------
// Greedy argmax keys (main.cpp:139-146: strict ">" from -1e10, lowest index
// on ties): a candidate is one 64-bit key, the order-preserving bits of the
// value above the complemented index, so the largest key is the largest
// value and, among equal values, the lowest index.  -0 is keyed as +0 (under
// ">" they are equal, so the lower index must win).  0 is "no candidate".
// ---------------------------------------------------------------------------
__device__ __forceinline__ unsigned long long argmax_key(float v, int i) {
    uint32_t b = __float_as_uint(v);
    if (b == 0x80000000u) b = 0u;
    uint32_t o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((unsigned long long)o << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)i);
}
__device__ __forceinline__ unsigned long long umax64(unsigned long long a, unsigned long long b) { return a > b ? a : b; }
__device__ __forceinline__ unsigned long long argmax_cand(float v, int i) { return v > -1e10f ? argmax_key(v, i) : 0ull; }
__device__ __forceinline__ int argmax_index(unsigned long long k) {
    return k ? (int)(0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFull)) : 0;
}

// ---------------------------------------------------------------------------
// host helpers
// ---------------------------------------------------------------------------

#define RINA_LAUNCH_CHECK()                                     \
    do {                                                        \
        if (hipGetLastError() != hipSuccess) return RINA_ERR_HIP; \
    } while (0)

static inline hipStream_t as_stream(void* s) { return (hipStream_t)s; }

// Number of compute units of the current device (cached per device).
int rina_num_cus();

// Scratch owned by the library, one buffer per (device, stream), grown on
// demand and never shrunk.  Used only where a caller aliases input and
// output, and for a norm that runs before a matvec as its own launch.
void* rina_scratch(size_t bytes, hipStream_t stream);

__device__ __forceinline__ int read_pos(int start_pos, const int* d_pos) {
    return start_pos + (d_pos ? *d_pos : 0);
}
