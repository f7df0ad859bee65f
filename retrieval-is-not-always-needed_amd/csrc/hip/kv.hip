// KV-cache block formats (q8_0 / q4_0 / q2_1 / q1_0), quantize-on-append
// fused with RoPE, and the Q4_0 / Q4_0F weight packers.
//
// Block rules follow rina-engine/src/kernels/quantize.cu:74-301 exactly
// (fp32 division, roundf, fp16 RNE scale); the q1_0 record is the
// documented 6 bytes [fp16 amax][u32 sign bits] of core/quant.h:44.
// Blocks are 2-byte aligned in every layout, so all stores are 16-bit.
#include "rina_common.hpp"
#include "kv_formats.hpp"

namespace {

// ---------------------------------------------------------------------------
// generic block quantize / dequantize (one thread per 32-value block)
// ---------------------------------------------------------------------------
__global__ void kv_quantize_kernel(int fmt, const float* __restrict__ src, uint8_t* __restrict__ dst, int64_t nb) {
    int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nb) return;
    float v[32];
    const float4* s4 = (const float4*)(src + b * 32);
#pragma unroll
    for (int i = 0; i < 8; i++) {
        float4 t = s4[i];
        v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
    }
    kvq::quantize_block(fmt, v, dst + b * kvq::block_bytes(fmt));
}

__global__ void kv_dequant_kernel(int fmt, const uint8_t* __restrict__ src, float* __restrict__ dst, int64_t n) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    int64_t b = i >> 5;
    dst[i] = kvq::dequant_one(fmt, src + b * kvq::block_bytes(fmt), (int)(i & 31));
}

// ---------------------------------------------------------------------------
// weight packers (tools/q4_pack.py:11-23,71-118)
// ---------------------------------------------------------------------------
__global__ void pack_q4_kernel(int fp32_scale, const float* __restrict__ src, uint8_t* __restrict__ dst, int64_t nb) {
    int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nb) return;
    const float* x = src + b * 32;
    float amax = 0.f;
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(x[i]));
    float scale = amax / 7.0f;
    if (scale < 1e-10f) scale = 1e-10f;
    uint32_t nib[4] = {0, 0, 0, 0};
    for (int i = 0; i < 32; i++) {
        float y = x[i] / scale;
        int sgn = (y > 0.f) - (y < 0.f);
        float fl = fminf(floorf(fabsf(y) + 0.5f), 7.0f);
        int q = (int)fl * sgn + 7;
        nib[i >> 3] |= (uint32_t)(q & 0xF) << ((i & 7) * 4);
    }
    // byte j = q[2j] | q[2j+1] << 4: nibble i sits at bit 4*(i%8) of dword i/8
    if (fp32_scale) {
        uint32_t* o = (uint32_t*)(dst + b * 20);
        o[0] = __float_as_uint(scale);
        o[1] = nib[0]; o[2] = nib[1]; o[3] = nib[2]; o[4] = nib[3];
    } else {
        uint16_t* o = (uint16_t*)(dst + b * 18);
        o[0] = (uint16_t)f32_to_f16_rne(scale);
        for (int d = 0; d < 4; d++) { o[1 + 2 * d] = (uint16_t)nib[d]; o[2 + 2 * d] = (uint16_t)(nib[d] >> 16); }
    }
}

// fp32 -> fp16 bits by truncation (src/loader_hf.cpp:208-216): top 10
// mantissa bits, biased exponent <= 0 -> signed zero, >= 31 -> 0x7FFF class.
__device__ __forceinline__ uint32_t f32_to_f16_trunc(float f) {
    const uint32_t p = __float_as_uint(f);
    const uint32_t sign = (p >> 31) & 1u;
    int exp = (int)((p >> 23) & 0xFFu) - 127 + 15;
    uint32_t mant = (p >> 13) & 0x3FFu;
    if (exp <= 0) { exp = 0; mant = 0; }
    else if (exp >= 31) { exp = 31; mant = 0x3FFu; }
    return (sign << 15) | ((uint32_t)exp << 10) | mant;
}

// HF-loader Q4_0 quantizer (src/loader_hf.cpp:196-230): scale = max(amax/7,
// 1e-10) over the block's present elements, q = clamp(roundf(x/scale), -7, 7)
// + 7, truncating fp16 scale; bytes of a short last block's missing
// elements stay zero.  One thread per block.
__global__ void pack_q4_hf_kernel(const float* __restrict__ src, uint8_t* __restrict__ dst, int64_t n, int64_t nb) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nb) return;
    const int64_t start = b * 32;
    const int cnt = (int)min((int64_t)32, n - start);
    float amax = 0.f;
    for (int i = 0; i < cnt; i++) amax = fmaxf(amax, fabsf(src[start + i]));
    float scale = amax / 7.0f;
    if (scale < 1e-10f) scale = 1e-10f;
    uint32_t nib[4] = {0, 0, 0, 0};
    for (int i = 0; i < cnt; i++) {
        int q = (int)roundf(src[start + i] / scale);
        q = min(max(q, -7), 7) + 7;
        nib[i >> 3] |= (uint32_t)(q & 0xF) << ((i & 7) * 4);
    }
    uint16_t* o = (uint16_t*)(dst + b * 18);
    o[0] = (uint16_t)f32_to_f16_trunc(scale);
    for (int d = 0; d < 4; d++) { o[1 + 2 * d] = (uint16_t)nib[d]; o[2 + 2 * d] = (uint16_t)(nib[d] >> 16); }
}

__global__ void dequant_weights_kernel(int qt, const uint8_t* __restrict__ w, float* __restrict__ out, int64_t n) {
    int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n) return;
    out[e] = kvq::weight_elem(qt, w, e);
}

// ---------------------------------------------------------------------------
// RoPE + quantize-on-append (gqa_layer.cu:147-190): one workgroup per token
// ---------------------------------------------------------------------------
struct AppendArgs {
    float* q; float* k; const float* v;
    const float* qc; const float* qs; const float* kc; const float* ks;
    uint8_t* ck; uint8_t* cv;
    int mode, pre_rope, T, H, Hkv, dh, start_pos, max_seq;
    const int* d_pos;
};

__global__ __launch_bounds__(256) void rope_append_kernel(AppendArgs a) {
    extern __shared__ float kl[];                 // [2][Hkv*dh]: raw, rotated
    const int t = blockIdx.x, tid = threadIdx.x;
    const int kvd = a.Hkv * a.dh, half = a.dh / 2;
    const int pos = read_pos(a.start_pos, a.d_pos) + t;
    // capacity guard (tables and cache hold max_seq rows; the host checks
    // host-known positions, this covers device positions)
    if (pos < 0 || pos >= a.max_seq) return;
    float* krow = a.k + (int64_t)t * kvd;
    float* qrow = a.q + (int64_t)t * a.H * a.dh;
    float* kraw = kl;
    float* krot = kl + kvd;
    for (int i = tid; i < kvd; i += blockDim.x) kraw[i] = krow[i];
    // q rotation: pairs (i, i+half) of each head (ops/rope.cu:125-149)
    if (a.qc) {
        for (int p = tid; p < a.H * half; p += blockDim.x) {
            int h = p / half, i = p % half;
            float c = a.qc[(int64_t)pos * half + i], s = a.qs[(int64_t)pos * half + i];
            float* r = qrow + h * a.dh;
            float x0 = r[i], x1 = r[i + half];
            r[i] = x0 * c - x1 * s;
            r[i + half] = x0 * s + x1 * c;
        }
    }
    __syncthreads();
    for (int p = tid; p < a.Hkv * half; p += blockDim.x) {
        int h = p / half, i = p % half;
        float x0 = kraw[h * a.dh + i], x1 = kraw[h * a.dh + i + half];
        if (a.kc) {
            float c = a.kc[(int64_t)pos * half + i], s = a.ks[(int64_t)pos * half + i];
            krot[h * a.dh + i] = x0 * c - x1 * s;
            krot[h * a.dh + i + half] = x0 * s + x1 * c;
        } else {
            krot[h * a.dh + i] = x0;
            krot[h * a.dh + i + half] = x1;
        }
    }
    __syncthreads();
    for (int i = tid; i < kvd; i += blockDim.x) krow[i] = krot[i];
    const float* kc_src = a.pre_rope ? kraw : krot;
    const float* vrow = a.v + (int64_t)t * kvd;
    if (a.mode == RINA_KV_FP32) {
        float* ck = (float*)a.ck + (int64_t)pos * kvd;
        float* cv = (float*)a.cv + (int64_t)pos * kvd;
        for (int i = tid; i < kvd; i += blockDim.x) { ck[i] = kc_src[i]; cv[i] = vrow[i]; }
        return;
    }
    int kf, vf;
    kvq::mode_formats(a.mode, kf, vf);
    const int64_t b0 = (int64_t)pos * (kvd / 32);
    // one value per thread, a half wave per 32-value block: 2*kvd is a
    // multiple of 64 and blockDim.x of 256, so every wave runs the loop's
    // iterations whole, and kvd is a multiple of 32, so no half wave holds
    // both K and V
    for (int e = tid; e < 2 * kvd; e += blockDim.x) {
        const bool isv = e >= kvd;
        const int i = isv ? e - kvd : e;
        const int64_t b = b0 + i / 32;
        if (isv) kvq::quantize_block_lanes(vf, vrow[i], a.cv + b * kvq::block_bytes(vf));
        else kvq::quantize_block_lanes(kf, kc_src[i], a.ck + b * kvq::block_bytes(kf));
    }
}

bool valid_kvf(int f) { return f >= RINA_KVF_Q8_0 && f <= RINA_KVF_Q1_0; }

}  // namespace

extern "C" int rina_hip_kv_quantize(int fmt, const float* src, void* dst, int64_t n, void* stream) {
    if (!valid_kvf(fmt)) return RINA_ERR_QTYPE;
    if (!src || !dst || n < 0) return RINA_ERR_ARG;
    if (n % 32 || (uintptr_t)src % 16 || (uintptr_t)dst % 2) return RINA_ERR_SHAPE;
    int64_t nb = n / 32;
    if (nb == 0) return RINA_OK;
    hipLaunchKernelGGL(kv_quantize_kernel, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, as_stream(stream), fmt, src,
                       (uint8_t*)dst, nb);
    RINA_LAUNCH_CHECK();
    return RINA_OK;
}

extern "C" int rina_hip_kv_dequant(int fmt, const void* src, float* dst, int64_t n, void* stream) {
    if (!valid_kvf(fmt)) return RINA_ERR_QTYPE;
    if (!src || !dst || n < 0) return RINA_ERR_ARG;
    if (n % 32 || (uintptr_t)src % 2) return RINA_ERR_SHAPE;
    if (n == 0) return RINA_OK;
    hipLaunchKernelGGL(kv_dequant_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, as_stream(stream), fmt,
                       (const uint8_t*)src, dst, n);
    RINA_LAUNCH_CHECK();
    return RINA_OK;
}

extern "C" size_t rina_hip_kv_region_bytes(int mode, int which_v, int max_seq, int kv_dim) {
    if (mode == RINA_KV_FP32) return (size_t)max_seq * kv_dim * 4;
    int kf, vf;
    if (!kvq::mode_formats_host(mode, kf, vf)) return 0;
    return (size_t)max_seq * (kv_dim / 32) * kvq::block_bytes_host(which_v ? vf : kf);
}

extern "C" int rina_hip_pack_weights(int qt, const float* src, int64_t n, void* dst, void* stream) {
    if (qt != RINA_QT_Q4_0 && qt != RINA_QT_Q4_0F) return RINA_ERR_QTYPE;
    if (!src || !dst || n < 0) return RINA_ERR_ARG;
    if (n % 32) return RINA_ERR_SHAPE;
    if ((uintptr_t)dst % (qt == RINA_QT_Q4_0F ? 4 : 2)) return RINA_ERR_ARG;
    int64_t nb = n / 32;
    if (nb == 0) return RINA_OK;
    hipLaunchKernelGGL(pack_q4_kernel, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, as_stream(stream),
                       qt == RINA_QT_Q4_0F ? 1 : 0, src, (uint8_t*)dst, nb);
    RINA_LAUNCH_CHECK();
    return RINA_OK;
}

extern "C" int rina_hip_pack_weights_hf(const float* src, int64_t n, void* dst, void* stream) {
    if (!src || !dst || n < 0) return RINA_ERR_ARG;
    if ((uintptr_t)dst % 2) return RINA_ERR_ARG;
    const int64_t nb = (n + 31) / 32;
    if (nb == 0) return RINA_OK;
    hipLaunchKernelGGL(pack_q4_hf_kernel, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, as_stream(stream), src,
                       (uint8_t*)dst, n, nb);
    RINA_LAUNCH_CHECK();
    return RINA_OK;
}

extern "C" int rina_hip_dequant_weights(int qt, const void* src, int64_t n, float* dst, void* stream) {
    if (qt != RINA_QT_Q4_0 && qt != RINA_QT_Q4_0F && qt != RINA_QT_GGML_Q2_K && qt != RINA_QT_FP32)
        return RINA_ERR_QTYPE;
    if (!src || !dst || n < 0) return RINA_ERR_ARG;
    if (n == 0) return RINA_OK;
    hipLaunchKernelGGL(dequant_weights_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, as_stream(stream), qt,
                       (const uint8_t*)src, dst, n);
    RINA_LAUNCH_CHECK();
    return RINA_OK;
}

extern "C" int rina_hip_rope_append(float* q, float* k, const float* v, const float* qc, const float* qs,
                                    const float* kc, const float* ks, void* cache_k, void* cache_v, int mode,
                                    int pre_rope, int T, int H, int Hkv, int dh, int start_pos, const int* d_pos,
                                    int max_seq, void* stream) {
    if (!q || !k || !v || !cache_k || !cache_v || T < 1 || H < 1 || Hkv < 1 || dh < 2 || (dh & 1)) return RINA_ERR_ARG;
    if (mode < RINA_KV_FP32 || mode > RINA_KV_Q2K_Q1V) return RINA_ERR_QTYPE;
    if (H % Hkv) return RINA_ERR_SHAPE;
    if (mode != RINA_KV_FP32 && (Hkv * dh) % 32) return RINA_ERR_SHAPE;
    if ((qc == nullptr) != (qs == nullptr) || (kc == nullptr) != (ks == nullptr)) return RINA_ERR_ARG;
    if (!d_pos && (start_pos < 0 || start_pos + T > max_seq)) return RINA_ERR_RANGE;
    AppendArgs a{q, k, v, qc, qs, kc, ks, (uint8_t*)cache_k, (uint8_t*)cache_v, mode, pre_rope, T, H, Hkv, dh,
                 start_pos, max_seq, d_pos};
    size_t lds = 2 * (size_t)Hkv * dh * 4;
    if (lds > 64 * 1024) return RINA_ERR_SHAPE;
    hipLaunchKernelGGL(rope_append_kernel, dim3(T), dim3(256), lds, as_stream(stream), a);
    RINA_LAUNCH_CHECK();
    return RINA_OK;
}
