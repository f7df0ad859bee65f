// Block codecs shared by the KV append, attention and weight kernels.
#pragma once
#include "rina_common.hpp"

namespace kvq {

__host__ __device__ constexpr int block_bytes_c(int fmt) {
    return fmt == RINA_KVF_Q8_0 ? 34 : fmt == RINA_KVF_Q4_0 ? 18 : fmt == RINA_KVF_Q2_1 ? 10 : fmt == RINA_KVF_Q1_0 ? 6 : 128;
}
__device__ __forceinline__ int block_bytes(int fmt) { return block_bytes_c(fmt); }
static inline int block_bytes_host(int fmt) { return block_bytes_c(fmt); }

// mode -> (K format, V format): rina-engine/src/core/buffer.cpp:104-113
__host__ __device__ inline bool mode_formats_hd(int mode, int& kf, int& vf) {
    switch (mode) {
        case RINA_KV_Q8: kf = RINA_KVF_Q8_0; vf = RINA_KVF_Q8_0; return true;
        case RINA_KV_Q4: kf = RINA_KVF_Q4_0; vf = RINA_KVF_Q4_0; return true;
        case RINA_KV_Q4K_Q2V: kf = RINA_KVF_Q4_0; vf = RINA_KVF_Q2_1; return true;
        case RINA_KV_Q2: kf = RINA_KVF_Q2_1; vf = RINA_KVF_Q2_1; return true;
        case RINA_KV_Q2K_Q1V: kf = RINA_KVF_Q2_1; vf = RINA_KVF_Q1_0; return true;
        default: kf = vf = 0; return false;
    }
}
__device__ __forceinline__ void mode_formats(int mode, int& kf, int& vf) { mode_formats_hd(mode, kf, vf); }
static inline bool mode_formats_host(int mode, int& kf, int& vf) { return mode_formats_hd(mode, kf, vf); }

__device__ __forceinline__ uint32_t ld16(const uint8_t* p) { return *(const uint16_t*)p; }
__device__ __forceinline__ void st16(uint8_t* p, uint32_t v) { *(uint16_t*)p = (uint16_t)v; }

// One 32-value block (kernels/quantize.cu:74-270).
__device__ inline void quantize_block(int fmt, const float* v, uint8_t* o) {
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i++) {
        float a = fabsf(v[i]);
        if (a > amax) amax = a;
    }
    if (fmt == RINA_KVF_Q8_0) {
        float scale = amax / 127.0f;
        if (scale < 1e-10f) scale = 1e-10f;
        st16(o, f32_to_f16_rne(scale));
#pragma unroll
        for (int i = 0; i < 32; i += 2) {
            int q0 = (int)roundf(v[i] / scale), q1 = (int)roundf(v[i + 1] / scale);
            q0 = min(max(q0, -127), 127);
            q1 = min(max(q1, -127), 127);
            st16(o + 2 + i, (uint32_t)(q0 & 0xFF) | ((uint32_t)(q1 & 0xFF) << 8));
        }
    } else if (fmt == RINA_KVF_Q4_0) {
        float scale = amax / 7.0f;
        if (scale < 1e-10f) scale = 1e-10f;
        st16(o, f32_to_f16_rne(scale));
#pragma unroll
        for (int j = 0; j < 16; j += 2) {
            uint32_t w = 0;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                int q = (int)roundf(v[2 * j + k] / scale);
                q = min(max(q, -7), 7) + 7;
                w |= (uint32_t)(q & 0xF) << (4 * k);
            }
            st16(o + 2 + j, w);
        }
    } else if (fmt == RINA_KVF_Q2_1) {
        st16(o, f32_to_f16_rne(amax));
        uint32_t d[4] = {0, 0, 0, 0};
        if (amax > 1e-10f) {
#pragma unroll
            for (int i = 0; i < 32; i++) {
                int q = (int)roundf(v[i] / amax);
                q = min(max(q, -1), 1) + 1;
                d[i >> 3] |= (uint32_t)(q & 3) << ((i & 7) * 2);   // byte i/4, shift 2(i%4)
            }
        }
#pragma unroll
        for (int k = 0; k < 4; k++) st16(o + 2 + 2 * k, d[k]);
    } else {  // RINA_KVF_Q1_0, 6-byte record
        st16(o, f32_to_f16_rne(amax));
        uint32_t bits = 0;
        if (amax > 1e-10f) {
#pragma unroll
            for (int i = 0; i < 32; i++) bits |= (v[i] > 0.0f ? 1u : 0u) << i;
        }
        st16(o + 2, bits & 0xFFFF);
        st16(o + 4, bits >> 16);
    }
}

// The same block quantized by a 32-lane half wave: lane (__lane_id() & 31) = i
// holds element i, all 32 lanes are active and pass the same fmt and o.
// The amax comes from a butterfly max (NaN and -0 enter as 0, as they
// drop out of the serial scan above), each lane applies quantize_block's
// per-element arithmetic to its own value (the same fp32 division and
// roundf), and the codes are OR-gathered into the 16-bit words the serial
// form stores, so the record bytes are identical.  Used where one thread
// per block would leave the rest of the workgroup idle (the decode appends).
__device__ inline void quantize_block_lanes(int fmt, float v, uint8_t* o) {
    const int i = (int)(__lane_id() & 31);
    const float av = fabsf(v);
    float amax = av > 0.f ? av : 0.f;
#pragma unroll
    for (int m = 1; m < 32; m <<= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 32));
    if (fmt == RINA_KVF_Q8_0) {
        float scale = amax / 127.0f;
        if (scale < 1e-10f) scale = 1e-10f;
        int q = (int)roundf(v / scale);
        q = min(max(q, -127), 127);
        uint32_t w = (uint32_t)(q & 0xFF) << (8 * (i & 1));
        w |= __shfl_xor(w, 1, 32);
        if (i == 0) st16(o, f32_to_f16_rne(scale));
        if ((i & 1) == 0) st16(o + 2 + i, w);
    } else if (fmt == RINA_KVF_Q4_0) {
        float scale = amax / 7.0f;
        if (scale < 1e-10f) scale = 1e-10f;
        int q = (int)roundf(v / scale);
        q = min(max(q, -7), 7) + 7;
        uint32_t w = (uint32_t)(q & 0xF) << (4 * (i & 3));
        w |= __shfl_xor(w, 1, 32);
        w |= __shfl_xor(w, 2, 32);
        if (i == 0) st16(o, f32_to_f16_rne(scale));
        if ((i & 3) == 0) st16(o + 2 + i / 2, w);
    } else if (fmt == RINA_KVF_Q2_1) {
        uint32_t c = 0;
        if (amax > 1e-10f) {
            int q = (int)roundf(v / amax);
            c = (uint32_t)((min(max(q, -1), 1) + 1) & 3);
        }
        uint32_t w = c << (2 * (i & 7));
        w |= __shfl_xor(w, 1, 32);
        w |= __shfl_xor(w, 2, 32);
        w |= __shfl_xor(w, 4, 32);
        if (i == 0) st16(o, f32_to_f16_rne(amax));
        if ((i & 7) == 0) st16(o + 2 + i / 4, w);
    } else {  // RINA_KVF_Q1_0
        uint32_t w = (amax > 1e-10f && v > 0.0f ? 1u : 0u) << (i & 15);
        w |= __shfl_xor(w, 1, 32);
        w |= __shfl_xor(w, 2, 32);
        w |= __shfl_xor(w, 4, 32);
        w |= __shfl_xor(w, 8, 32);
        if (i == 0) st16(o, f32_to_f16_rne(amax));
        if ((i & 15) == 0) st16(o + 2 + i / 8, w);
    }
}

// Element i of one block (kernels/quantize.cu:106-295).
__device__ __forceinline__ float dequant_one(int fmt, const uint8_t* b, int i) {
    float s = f16_to_f32(ld16(b));
    if (fmt == RINA_KVF_Q8_0) return (float)(int8_t)b[2 + i] * s;
    if (fmt == RINA_KVF_Q4_0) return (float)((int)((b[2 + (i >> 1)] >> ((i & 1) * 4)) & 0xF) - 7) * s;
    if (fmt == RINA_KVF_Q2_1) return (float)((int)((b[2 + (i >> 2)] >> ((i & 3) * 2)) & 3) - 1) * s;
    uint32_t bits = ld16(b + 2) | (ld16(b + 4) << 16);
    return ((bits >> i) & 1u) ? s : -s;
}

// Weight element e of a packed stream (flat order): ops/linear.cu:77-81,
// :115-119 (Q4_0 / Q4_0F), :413-431 (Q2_K flat indexing).
__device__ __forceinline__ float weight_elem(int qt, const uint8_t* w, int64_t e) {
    if (qt == RINA_QT_Q4_0) {
        const uint8_t* b = w + (e >> 5) * 18;
        int i = (int)(e & 31);
        return (float)((int)((b[2 + (i >> 1)] >> ((i & 1) * 4)) & 0xF) - 7) * f16_to_f32(ld16(b));
    }
    if (qt == RINA_QT_Q4_0F) {
        const uint8_t* b = w + (e >> 5) * 20;
        int i = (int)(e & 31);
        return (float)((int)((b[4 + (i >> 1)] >> ((i & 1) * 4)) & 0xF) - 7) * __uint_as_float(*(const uint32_t*)b);
    }
    if (qt == RINA_QT_GGML_Q2_K) {
        const uint8_t* bd = w + (e >> 8) * 84;
        int inb = (int)(e & 255);
        int page = inb >> 7, pos = inb & 127, l = pos & 31, g = pos >> 5;
        uint32_t sc = bd[8 * page + l / 16 + 2 * g];
        float dall = f16_to_f32(ld16(bd + 80)), dmin = f16_to_f32(ld16(bd + 82));
        int q = (bd[16 + 32 * page + l] >> (2 * g)) & 3;
        return fmaf(dall * (float)(sc & 0xF), (float)q, -(dmin * (float)(sc >> 4)));
    }
    return ((const float*)w)[e];
}

}  // namespace kvq
