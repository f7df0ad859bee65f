/*
 * rina_oracle.c — CPU restatement of the RINA engine decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY (the parity checker; never part of the product).
 * Built with -ffp-contract=off: every FMA the reference's nvcc build would
 * form (default --fmad=true) is written as fmaf() here, every other
 * product/sum rounds separately.  Reference paths are relative to
 * rina-engine/src/ unless stated otherwise.
 */
#include "rina_oracle.h"
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* ------------------------------------------------------------------ */
/* fp16                                                                */
/* ------------------------------------------------------------------ */

/* IEEE-754 binary32 -> binary16, round to nearest even, subnormals kept,
 * overflow to inf, NaN kept quiet.  This is __float2half, used by the KV
 * quantizers (kernels/quantize.cu:89,148,204,263) and by struct.pack('<e')
 * in tools/q4_pack.py:89 (exact fp32 promoted to double, then RNE). */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {
        if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
        return (uint16_t)(sign | 0x7c00u);
    }
    int e = (int)(ax >> 23) - 127;
    uint32_t mant = ax & 0x7fffffu;
    if (e > 15) return (uint16_t)(sign | 0x7c00u);
    if (e >= -14) {
        uint32_t h = ((uint32_t)(e + 15) << 10) | (mant >> 13);
        uint32_t rem = mant & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;   /* may carry into inf */
        return (uint16_t)(sign | h);
    }
    /* f16 subnormal: value in units of 2^-24 is m * 2^(e+1) */
    if (ax == 0) return (uint16_t)sign;
    uint32_t m = mant | (e == -127 ? 0u : 0x800000u);
    if (e == -127) e = -126;  /* f32 subnormal input */
    int s = -(e + 1);
    if (s > 24) return (uint16_t)sign;
    uint32_t r = m >> s;
    uint32_t rem = m & ((1u << s) - 1u);
    uint32_t half = 1u << (s - 1);
    if (rem > half || (rem == half && (r & 1u))) r++;
    return (uint16_t)(sign | r);
}

/* src/loader_hf.cpp:208-216: keep the top 10 mantissa bits, flush
 * exponent <= 0 to signed zero and exponent >= 31 to 0x7FFF-class. */
uint16_t orc_f32_to_f16_trunc(float f) {
    uint32_t p;
    memcpy(&p, &f, 4);
    uint32_t sign = (p >> 31) & 1u;
    int32_t exp = (int32_t)((p >> 23) & 0xFFu) - 127 + 15;
    uint32_t mant = (p >> 13) & 0x3FFu;
    if (exp <= 0) { exp = 0; mant = 0; }
    else if (exp >= 31) { exp = 31; mant = 0x3FF; }
    return (uint16_t)((sign << 15) | ((uint32_t)exp << 10) | mant);
}

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) x = sign;
        else {                       /* subnormal: normalize */
            int k = 0;
            while (!(m & 0x400u)) { m <<= 1; k++; }
            m &= 0x3ffu;
            x = sign | ((uint32_t)(127 - 15 + 1 - k) << 23) | (m << 13);
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e - 15 + 127) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

static inline float ld_f16(const uint8_t* p) {
    uint16_t h = (uint16_t)(p[0] | (p[1] << 8));
    return orc_f16_to_f32(h);
}
static inline void st_f16(uint8_t* p, uint16_t h) { p[0] = (uint8_t)(h & 0xff); p[1] = (uint8_t)(h >> 8); }
static inline float ld_f32(const uint8_t* p) { float f; memcpy(&f, p, 4); return f; }

/* ------------------------------------------------------------------ */
/* weight formats                                                      */
/* ------------------------------------------------------------------ */

/* core/quant.h:75-86 */
size_t orc_quantized_size(int64_t n, int qt) {
    switch (qt) {
        case ORC_Q4_0:  return (size_t)((n + 31) / 32) * 18;
        case ORC_Q4_0F: return (size_t)((n + 31) / 32) * 20;
        case ORC_Q2_1:  return (size_t)((n + 31) / 32) * 10;
        case ORC_Q1_0:  return (size_t)((n + 31) / 32) * 6;
        case ORC_GGML_Q2_K: return (size_t)((n + 255) / 256) * 84;
        default: return (size_t)n * 4;
    }
}

/* tools/q4_pack.py:71-78 (_quantize_blocks): q = sign(y)*clamp(floor(|y|+0.5),0,7),
 * y = x/scale in fp32; stored nibble q+7. */
static void q4_block_nibbles(const float* x, float scale, uint8_t* data16) {
    memset(data16, 0, 16);
    for (int i = 0; i < 32; i++) {
        float y = x[i] / scale;
        int sgn = (y > 0.0f) - (y < 0.0f);
        float fl = floorf(fabsf(y) + 0.5f);
        if (fl < 0.0f) fl = 0.0f;
        if (fl > 7.0f) fl = 7.0f;
        int q = (int)fl * sgn;
        if (q < -7) q = -7;
        if (q > 7) q = 7;
        int qu = q + 7;
        data16[i >> 1] |= (uint8_t)((qu & 0xF) << ((i & 1) * 4));   /* q4_pack.py:83-85 */
    }
}

static float q4_block_scale(const float* x) {
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) { float a = fabsf(x[i]); if (a > amax) amax = a; }
    float scale = amax / 7.0f;            /* q4_pack.py:19-20 */
    if (scale < 1e-10f) scale = 1e-10f;   /* clamp(min=1e-10) */
    return scale;
}

/* tools/q4_pack.py:11-23 + _pack_blocks_q4_0 :80-92 (fp16 RNE scale) */
void orc_pack_q4_0(const float* x, int64_t n, uint8_t* out) {
    int64_t nb = n / 32;
    for (int64_t b = 0; b < nb; b++) {
        const float* xb = x + b * 32;
        uint8_t* o = out + b * 18;
        float scale = q4_block_scale(xb);
        st_f16(o, orc_f32_to_f16(scale));
        q4_block_nibbles(xb, scale, o + 2);
    }
}

/* tools/q4_pack.py:95-118 (fp32 scale, 20 B blocks) */
void orc_pack_q4_0f(const float* x, int64_t n, uint8_t* out) {
    int64_t nb = n / 32;
    for (int64_t b = 0; b < nb; b++) {
        const float* xb = x + b * 32;
        uint8_t* o = out + b * 20;
        float scale = q4_block_scale(xb);
        memcpy(o, &scale, 4);
        q4_block_nibbles(xb, scale, o + 4);
    }
}

/* src/loader_hf.cpp:196-230: roundf, truncating fp16 scale, a short last
 * block keeps zero bytes for the missing elements. */
void orc_pack_q4_0_hf(const float* x, int64_t n, uint8_t* out) {
    int64_t nb = (n + 31) / 32;
    memset(out, 0, (size_t)nb * 18);
    for (int64_t b = 0; b < nb; b++) {
        int64_t start = b * 32, end = start + 32 < n ? start + 32 : n;
        float amax = 0.0f;
        for (int64_t i = start; i < end; i++) { float a = fabsf(x[i]); amax = amax > a ? amax : a; }
        float scale = amax / 7.0f;
        if (scale < 1e-10f) scale = 1e-10f;
        st_f16(out + b * 18, orc_f32_to_f16_trunc(scale));
        for (int64_t i = start; i < end; i++) {
            float qf = x[i] / scale;
            int qi = (int)roundf(qf);
            if (qi < -7) qi = -7;
            if (qi > 7) qi = 7;
            int qu = qi + 7;
            int idx = (int)(i - start);
            uint8_t* byte = out + b * 18 + 2 + idx / 2;
            if (idx % 2 == 0) *byte = (uint8_t)((*byte & 0xF0) | (qu & 0x0F));
            else *byte = (uint8_t)((*byte & 0x0F) | ((qu & 0x0F) << 4));
        }
    }
}

/* Q2_K element e of the flat stream: ops/linear.cu:406-431 (and the same
 * rule in :322-338 and ops/embedding.cu:72-101). */
static inline float q2k_value(const uint8_t* w, int64_t elem) {
    int64_t blk = elem / 256;
    int in_blk = (int)(elem % 256);
    const uint8_t* bd = w + blk * 84;
    float dall = ld_f16(bd + 80);
    float dmin = ld_f16(bd + 82);
    int page = in_blk / 128, pos = in_blk % 128;
    int l = pos % 32, g = pos / 32;
    int is = 8 * page + l / 16;
    uint8_t sc = bd[is + g * 2];
    float scale_val = dall * (float)(sc & 0xF);
    float min_val = dmin * (float)(sc >> 4);
    int q = (bd[16 + page * 32 + l] >> (g * 2)) & 3;
    return fmaf(scale_val, (float)q, -min_val);  /* exact products: one rounding */
}

/* Elements e0 .. e0+n-1 of the flat Q2_K stream, q2k_value's arithmetic
 * with each block's fp16 fields and 16 scale / min products formed once. */
static void q2k_range(const uint8_t* w, int64_t e0, int64_t n, float* out) {
    int64_t e = e0;
    const int64_t end = e0 + n;
    while (e < end) {
        const int64_t blk = e / 256;
        const int in0 = (int)(e - blk * 256);
        const int in1 = end - blk * 256 < 256 ? (int)(end - blk * 256) : 256;
        const uint8_t* bd = w + blk * 84;
        if (in0 == 0 && in1 == 256) {
            const float dall = ld_f16(bd + 80), dmin = ld_f16(bd + 82);
            float sv[16], mv[16];
            for (int i = 0; i < 16; i++) {
                sv[i] = dall * (float)(bd[i] & 0xF);
                mv[i] = dmin * (float)(bd[i] >> 4);
            }
            /* the same elements in runs of 16 that share one scale byte */
            for (int page = 0; page < 2; page++)
                for (int g = 0; g < 4; g++)
                    for (int half = 0; half < 2; half++) {
                        const int is = 8 * page + half + 2 * g;
                        const float sc = sv[is], mn = -mv[is];
                        const uint8_t* qs = bd + 16 + page * 32 + half * 16;
                        float* o = out + page * 128 + g * 32 + half * 16;
                        for (int l = 0; l < 16; l++) o[l] = fmaf(sc, (float)((qs[l] >> (2 * g)) & 3), mn);
                    }
            out += 256;
        } else {
            for (int j = in0; j < in1; j++) *out++ = q2k_value(w, blk * 256 + j);
        }
        e = blk * 256 + in1;
    }
}

static inline float q4_value(const uint8_t* blk, int i, float scale, int off) {
    int q = (blk[off + (i >> 1)] >> ((i & 1) << 2)) & 0xF;
    return (float)(q - 7) * scale;
}

void orc_dequant_weights(const void* wv, int qt, int64_t n, float* out) {
    const uint8_t* w = (const uint8_t*)wv;
    switch (qt) {
        case ORC_Q4_0:
            for (int64_t e = 0; e < n; e++) {
                const uint8_t* b = w + (e / 32) * 18;
                out[e] = q4_value(b, (int)(e % 32), ld_f16(b), 2);
            }
            break;
        case ORC_Q4_0F:
            for (int64_t e = 0; e < n; e++) {
                const uint8_t* b = w + (e / 32) * 20;
                out[e] = q4_value(b, (int)(e % 32), ld_f32(b), 4);
            }
            break;
        case ORC_GGML_Q2_K:
            q2k_range(w, 0, n, out);
            break;
        default:
            memcpy(out, wv, (size_t)n * 4);
    }
}

/* ------------------------------------------------------------------ */
/* matvec                                                              */
/* ------------------------------------------------------------------ */

int orc_num_threads(void) {
    const char* e = getenv("RINA_ORACLE_THREADS");
    if (e && atoi(e) > 0) return atoi(e);
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    return n > 0 ? (int)n : 1;
}

/* Row n of W dequantized to fp32 with the reference's per-element rule:
 * ops/linear.cu:77-81 (Q4_0), :115-119 (Q4_0F), :413-431 (Q2_K, flat
 * element index n*K+i), kernels/linear_fp32.cu:10-11 (FP32). */
static void weight_row(const uint8_t* w, int qt, int64_t n, int K, float* row) {
    switch (qt) {
        case ORC_Q4_0: {
            int nbk = K / 32;
            const uint8_t* r = w + n * nbk * 18;
            for (int b = 0; b < nbk; b++) {
                float scale = ld_f16(r + b * 18);
                for (int i = 0; i < 32; i++) row[b * 32 + i] = q4_value(r + b * 18, i, scale, 2);
            }
            break;
        }
        case ORC_Q4_0F: {
            int nbk = K / 32;
            const uint8_t* r = w + n * nbk * 20;
            for (int b = 0; b < nbk; b++) {
                float scale = ld_f32(r + b * 20);
                for (int i = 0; i < 32; i++) row[b * 32 + i] = q4_value(r + b * 20, i, scale, 4);
            }
            break;
        }
        case ORC_GGML_Q2_K: {
            q2k_range(w, n * (int64_t)K, K, row);
            break;
        }
        default:
            memcpy(row, (const float*)w + n * (int64_t)K, (size_t)K * 4);
    }
}

typedef struct {
    const uint8_t* w; int qt; const float* in; float* out;
    int M, N, K, t, nt;
} lin_job;

/* Each output is one serial K-loop `sum += deq(w) * in` (the reference's
 * per-thread loop, FMA-contracted): out[m,n] = fma chain over k in order.
 * Up to 8 rows m share one dequantized weight row (independent chains). */
static void* lin_worker(void* arg) {
    lin_job* j = (lin_job*)arg;
    int64_t per = ((int64_t)j->N + j->nt - 1) / j->nt;
    int64_t a = per * j->t, b = a + per < j->N ? a + per : j->N;
    const int K = j->K;
    if (j->M == 1) {
        /* four rows at a time: four independent chains, each in k order */
        float* rows = (float*)malloc((size_t)K * 4 * 4);
        const float* x = j->in;
        for (int64_t n = a; n < b; n += 4) {
            const int nr = b - n < 4 ? (int)(b - n) : 4;
            for (int r = 0; r < nr; r++) weight_row(j->w, j->qt, n + r, K, rows + (size_t)r * K);
            if (nr == 4) {
                float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
                const float *r0 = rows, *r1 = rows + K, *r2 = rows + 2 * (size_t)K, *r3 = rows + 3 * (size_t)K;
                for (int k = 0; k < K; k++) {
                    const float xv = x[k];
                    a0 = fmaf(r0[k], xv, a0);
                    a1 = fmaf(r1[k], xv, a1);
                    a2 = fmaf(r2[k], xv, a2);
                    a3 = fmaf(r3[k], xv, a3);
                }
                j->out[n] = a0; j->out[n + 1] = a1; j->out[n + 2] = a2; j->out[n + 3] = a3;
            } else {
                for (int r = 0; r < nr; r++) {
                    float acc = 0.f;
                    const float* rr = rows + (size_t)r * K;
                    for (int k = 0; k < K; k++) acc = fmaf(rr[k], x[k], acc);
                    j->out[n + r] = acc;
                }
            }
        }
        free(rows);
        return NULL;
    }
    float* row = (float*)malloc((size_t)j->K * 4);
    for (int64_t n = a; n < b; n++) {
        weight_row(j->w, j->qt, n, K, row);
        for (int m0 = 0; m0 < j->M; m0 += 8) {
            int mb = j->M - m0 < 8 ? j->M - m0 : 8;
            float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            const float* x[8];
            for (int i = 0; i < mb; i++) x[i] = j->in + (int64_t)(m0 + i) * K;
            if (mb == 8) {
                for (int k = 0; k < K; k++) {
                    float wv = row[k];
                    for (int i = 0; i < 8; i++) acc[i] = fmaf(wv, x[i][k], acc[i]);
                }
            } else {
                for (int k = 0; k < K; k++) {
                    float wv = row[k];
                    for (int i = 0; i < mb; i++) acc[i] = fmaf(wv, x[i][k], acc[i]);
                }
            }
            for (int i = 0; i < mb; i++) j->out[(int64_t)(m0 + i) * j->N + n] = acc[i];
        }
    }
    free(row);
    return NULL;
}

/* ops/linear.cu:140-167 dispatch, computed out of place */
int orc_linear(const void* w, int qt, const float* in, float* out, int M, int N, int K, int nthreads) {
    if (qt != ORC_Q4_0 && qt != ORC_Q4_0F && qt != ORC_GGML_Q2_K && qt != ORC_FP32) return -1;
    if ((qt == ORC_Q4_0 || qt == ORC_Q4_0F) && (K % 32)) return -2;
    int nt = nthreads > 0 ? nthreads : orc_num_threads();
    int64_t total = (int64_t)M * N;
    if ((int64_t)N * K < 65536) nt = 1;
    if (nt > N) nt = N;
    if (nt > 256) nt = 256;
    float* tmp = (in == out) ? (float*)malloc((size_t)total * 4) : out;
    lin_job jobs[256];
    pthread_t th[256];
    for (int t = 0; t < nt; t++) {
        jobs[t] = (lin_job){(const uint8_t*)w, qt, in, tmp, M, N, K, t, nt};
        if (nt > 1) pthread_create(&th[t], NULL, lin_worker, &jobs[t]);
        else lin_worker(&jobs[t]);
    }
    if (nt > 1) for (int t = 0; t < nt; t++) pthread_join(th[t], NULL);
    if (tmp != out) { memcpy(out, tmp, (size_t)total * 4); free(tmp); }
    return 0;
}

/* ------------------------------------------------------------------ */
/* KV cache block formats (kernels/quantize.cu)                        */
/* ------------------------------------------------------------------ */

int orc_kv_block_bytes(int fmt) {
    switch (fmt) {
        case ORC_KVF_Q8_0: return 34;
        case ORC_KVF_Q4_0: return 18;
        case ORC_KVF_Q2_1: return 10;
        case ORC_KVF_Q1_0: return 6;   /* documented record: core/quant.h:44 */
        default: return 128;           /* fp32: 32 floats */
    }
}

/* buffer.cpp:104-113 mode -> (K format, V format) */
void orc_kv_mode_formats(int mode, int* kf, int* vf) {
    switch (mode) {
        case ORC_KV_Q8: *kf = ORC_KVF_Q8_0; *vf = ORC_KVF_Q8_0; break;
        case ORC_KV_Q4: *kf = ORC_KVF_Q4_0; *vf = ORC_KVF_Q4_0; break;
        case ORC_KV_Q4K_Q2V: *kf = ORC_KVF_Q4_0; *vf = ORC_KVF_Q2_1; break;
        case ORC_KV_Q2: *kf = ORC_KVF_Q2_1; *vf = ORC_KVF_Q2_1; break;
        case ORC_KV_Q2K_Q1V: *kf = ORC_KVF_Q2_1; *vf = ORC_KVF_Q1_0; break;
        default: *kf = 0; *vf = 0;
    }
}

static float amax32(const float* x) {
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) { float a = fabsf(x[i]); if (a > amax) amax = a; }
    return amax;
}

void orc_kv_quantize(int fmt, const float* in, void* outv, int64_t n) {
    uint8_t* out = (uint8_t*)outv;
    int64_t nb = n / 32;
    for (int64_t b = 0; b < nb; b++) {
        const float* x = in + b * 32;
        float amax = amax32(x);
        switch (fmt) {
            case ORC_KVF_Q8_0: {           /* quantize.cu:248-270 */
                uint8_t* o = out + b * 34;
                float scale = amax / 127.0f;
                if (scale < 1e-10f) scale = 1e-10f;
                st_f16(o, orc_f32_to_f16(scale));
                for (int i = 0; i < 32; i++) {
                    int q = (int)roundf(x[i] / scale);
                    if (q < -127) q = -127;
                    if (q > 127) q = 127;
                    o[2 + i] = (uint8_t)(int8_t)q;
                }
                break;
            }
            case ORC_KVF_Q4_0: {           /* quantize.cu:188-214 */
                uint8_t* o = out + b * 18;
                float scale = amax / 7.0f;
                if (scale < 1e-10f) scale = 1e-10f;
                st_f16(o, orc_f32_to_f16(scale));
                memset(o + 2, 0, 16);
                for (int i = 0; i < 32; i++) {
                    int q = (int)roundf(x[i] / scale);
                    if (q < -7) q = -7;
                    if (q > 7) q = 7;
                    o[2 + i / 2] |= (uint8_t)(((q + 7) & 0xF) << ((i & 1) * 4));
                }
                break;
            }
            case ORC_KVF_Q2_1: {           /* quantize.cu:74-103 */
                uint8_t* o = out + b * 10;
                st_f16(o, orc_f32_to_f16(amax));
                memset(o + 2, 0, 8);
                if (amax > 1e-10f) {
                    for (int i = 0; i < 32; i++) {
                        int q = (int)roundf(x[i] / amax);
                        if (q < -1) q = -1;
                        if (q > 1) q = 1;
                        q += 1;
                        o[2 + i / 4] |= (uint8_t)((q & 3) << ((i % 4) * 2));
                    }
                }
                break;
            }
            case ORC_KVF_Q1_0: {           /* quantize.cu:136-157, 6 B record */
                uint8_t* o = out + b * 6;
                st_f16(o, orc_f32_to_f16(amax));
                uint32_t bits = 0;
                if (amax > 1e-10f)
                    for (int i = 0; i < 32; i++) if (x[i] > 0.0f) bits |= (1u << i);
                o[2] = (uint8_t)bits; o[3] = (uint8_t)(bits >> 8);
                o[4] = (uint8_t)(bits >> 16); o[5] = (uint8_t)(bits >> 24);
                break;
            }
        }
    }
}

void orc_kv_dequant(int fmt, const void* inv, float* out, int64_t n) {
    const uint8_t* in = (const uint8_t*)inv;
    int64_t nb = n / 32;
    for (int64_t b = 0; b < nb; b++) {
        float* y = out + b * 32;
        switch (fmt) {
            case ORC_KVF_Q8_0: {           /* quantize.cu:280-295 */
                const uint8_t* o = in + b * 34;
                float s = ld_f16(o);
                for (int i = 0; i < 32; i++) y[i] = (float)(int8_t)o[2 + i] * s;
                break;
            }
            case ORC_KVF_Q4_0: {           /* quantize.cu:224-239 */
                const uint8_t* o = in + b * 18;
                float s = ld_f16(o);
                for (int i = 0; i < 32; i++) y[i] = (float)(((o[2 + i / 2] >> ((i & 1) * 4)) & 0xF) - 7) * s;
                break;
            }
            case ORC_KVF_Q2_1: {           /* quantize.cu:112-127 */
                const uint8_t* o = in + b * 10;
                float s = ld_f16(o);
                for (int i = 0; i < 32; i++) y[i] = (float)(((o[2 + i / 4] >> ((i % 4) * 2)) & 3) - 1) * s;
                break;
            }
            case ORC_KVF_Q1_0: {           /* quantize.cu:166-179 */
                const uint8_t* o = in + b * 6;
                float s = ld_f16(o);
                uint32_t bits = (uint32_t)o[2] | ((uint32_t)o[3] << 8) | ((uint32_t)o[4] << 16) | ((uint32_t)o[5] << 24);
                for (int i = 0; i < 32; i++) y[i] = (bits & (1u << i)) ? s : -s;
                break;
            }
        }
    }
}

/* ------------------------------------------------------------------ */
/* glue                                                                */
/* ------------------------------------------------------------------ */

void orc_rms_norm(float* x, const float* w, int n, int d, float eps) {
    for (int r = 0; r < n; r++) {
        float* row = x + (int64_t)r * d;
        float ss = 0.0f;
        for (int i = 0; i < d; i++) ss = fmaf(row[i], row[i], ss);
        float inv = 1.0f / sqrtf(ss / (float)d + eps);
        for (int i = 0; i < d; i++) row[i] = row[i] * inv * w[i];
    }
}

/* Welford mean/var, biased variance, (x-mean)*rsqrt(var+eps)*gamma */
void orc_layer_norm(float* x, const float* w, int n, int d, float eps) {
    for (int r = 0; r < n; r++) {
        float* row = x + (int64_t)r * d;
        float m = 0.0f, m2 = 0.0f, c = 0.0f;
        for (int i = 0; i < d; i++) {
            float v = row[i];
            c += 1.0f;
            float dd = v - m;
            m += dd / c;
            m2 = fmaf(dd, v - m, m2);
        }
        float inv = 1.0f / sqrtf(m2 / (float)d + eps);
        for (int i = 0; i < d; i++) row[i] = (row[i] - m) * inv * (w ? w[i] : 1.0f);
    }
}

void orc_rope_neox(float* x, const float* ct, const float* st, int T, int H, int d, int start_pos) {
    int half = d / 2;
    for (int t = 0; t < T; t++)
        for (int h = 0; h < H; h++) {
            float* row = x + ((int64_t)t * H + h) * d;
            int p = start_pos + t;
            for (int i = 0; i < half; i++) {
                float c = ct[(int64_t)p * half + i], s = st[(int64_t)p * half + i];
                float x0 = row[i], x1 = row[i + half];
                row[i] = fmaf(x0, c, -(x1 * s));
                row[i + half] = fmaf(x0, s, x1 * c);
            }
        }
}

void orc_rope_hf(float* x, const float* ct, const float* st, int T, int H, int d, int start_pos) {
    int half = d / 2;
    for (int t = 0; t < T; t++)
        for (int h = 0; h < H; h++) {
            float* row = x + ((int64_t)t * H + h) * d;
            int p = start_pos + t;
            for (int i = 0; i < half; i++) {
                float c = ct[(int64_t)p * half + i], s = st[(int64_t)p * half + i];
                float x0 = row[2 * i], x1 = row[2 * i + 1];
                row[2 * i] = fmaf(x0, c, -(x1 * s));
                row[2 * i + 1] = fmaf(x0, s, x1 * c);
            }
        }
}

void orc_embedding(const void* wv, int qt, const int* ids, float* out, int n, int d) {
    const uint8_t* w = (const uint8_t*)wv;
    for (int t = 0; t < n; t++) {
        int id = ids[t] < 0 ? 0 : ids[t];
        float* o = out + (int64_t)t * d;
        switch (qt) {
            case ORC_Q4_0: orc_dequant_weights(w + (int64_t)id * (d / 32) * 18, ORC_Q4_0, d, o); break;
            case ORC_Q4_0F: orc_dequant_weights(w + (int64_t)id * (d / 32) * 20, ORC_Q4_0F, d, o); break;
            case ORC_GGML_Q2_K: /* row-aligned blocks: ops/embedding.cu:80-81 */
                orc_dequant_weights(w + (int64_t)id * ((d + 255) / 256) * 84, ORC_GGML_Q2_K, d, o); break;
            default: memcpy(o, (const float*)wv + (int64_t)id * d, (size_t)d * 4);
        }
    }
}

void orc_silu_mul(float* o, const float* g, const float* u, int n) {
    for (int i = 0; i < n; i++) o[i] = (g[i] / (1.0f + expf(-g[i]))) * u[i];
}
void orc_add(float* c, const float* a, const float* b, int n) { for (int i = 0; i < n; i++) c[i] = a[i] + b[i]; }
void orc_saxpy(float* d, const float* s, float p, int n) { for (int i = 0; i < n; i++) d[i] = fmaf(p, s[i], d[i]); }

int orc_argmax(const float* x, int n) {
    float mx = -1e10f;
    int am = 0;
    for (int i = 0; i < n; i++) if (x[i] > mx) { mx = x[i]; am = i; }
    return am;
}

/* ------------------------------------------------------------------ */
/* attention                                                           */
/* ------------------------------------------------------------------ */

/* kernels/flash_fp32.cu:12-94, one query row at a time, keys in order */
void orc_attn_rows(const float* q, int ldq, const float* k, int ldk,
                   const float* v, int ldv, float* o, int ldo,
                   int q0, int nq, int dq, int dh) {
    float rs = 1.0f / sqrtf((float)dq);
    for (int i = 0; i < nq; i++) {
        int qi = q0 + i;
        const float* qp = q + (int64_t)i * ldq;
        float* op = o + (int64_t)i * ldo;
        for (int d = 0; d < dh; d++) op[d] = 0.0f;
        float m = -1e10f, l = 0.0f, m_row = -1e10f;
        for (int kj = 0; kj <= qi; kj++) {
            const float* kp = k + (int64_t)kj * ldk;
            float dot = 0.0f;
            for (int d = 0; d < dq; d++) dot = fmaf(qp[d], kp[d], dot);
            float s = dot * rs;
            float old_l = l;
            float new_m = fmaxf(m, s);
            l = fmaf(l, expf(m - new_m), expf(s - new_m));
            m = new_m;
            float scale_old = old_l * expf(m_row - m) / l;
            float scale_new = expf(s - m) / l;
            const float* vp = v + (int64_t)kj * ldv;
            for (int d = 0; d < dh; d++) op[d] = fmaf(op[d], scale_old, vp[d] * scale_new);
            m_row = m;
        }
    }
}

typedef struct {
    const float *q, *ek, *ev;
    float* out;
    int H, rep, dh, kvd, start_pos, T, w, nw;
} gqa_head_job;

/* heads w, w + nw, ... of orc_gqa_attention (heads are independent) */
static void* gqa_head_worker(void* arg) {
    gqa_head_job* j = (gqa_head_job*)arg;
    for (int h = j->w; h < j->H; h += j->nw) {
        int kvh = h / j->rep;   /* build_qkv_fp32.cu:16 */
        orc_attn_rows(j->q + (int64_t)h * j->dh, j->H * j->dh, j->ek + (int64_t)kvh * j->dh, j->kvd,
                      j->ev + (int64_t)kvh * j->dh, j->kvd, j->out + (int64_t)h * j->dh, j->H * j->dh,
                      j->start_pos, j->T, j->dh, j->dh);
    }
    return NULL;
}

static void gqa_attention_nt(const float* q, const float* kcur, const float* vcur,
                             const float* k_cache, const float* v_cache,
                             const uint8_t* kq, const uint8_t* vq, int mode, int pre_rope,
                             const float* rkc, const float* rks,
                             int T, int start_pos, int H, int Hkv, int dh, float* out, int nt);

void orc_gqa_attention(const float* q, const float* kcur, const float* vcur,
                       const float* k_cache, const float* v_cache,
                       const uint8_t* kq, const uint8_t* vq, int mode, int pre_rope,
                       const float* rkc, const float* rks,
                       int T, int start_pos, int H, int Hkv, int dh, float* out) {
    gqa_attention_nt(q, kcur, vcur, k_cache, v_cache, kq, vq, mode, pre_rope, rkc, rks, T, start_pos, H, Hkv, dh, out,
                     1);
}

static void gqa_attention_nt(const float* q, const float* kcur, const float* vcur,
                             const float* k_cache, const float* v_cache,
                             const uint8_t* kq, const uint8_t* vq, int mode, int pre_rope,
                             const float* rkc, const float* rks,
                             int T, int start_pos, int H, int Hkv, int dh, float* out, int nt) {
    int kvd = Hkv * dh;
    int total = start_pos + T;
    /* ext_k / ext_v of gqa_layer.cu:204-244: cached rows [0,start_pos) in fp32,
     * then the current rows in fp32 */
    float* ek = (float*)malloc((size_t)total * kvd * 4);
    float* ev = (float*)malloc((size_t)total * kvd * 4);
    if (start_pos > 0) {
        if (mode == ORC_KV_FP32) {
            memcpy(ek, k_cache, (size_t)start_pos * kvd * 4);
            memcpy(ev, v_cache, (size_t)start_pos * kvd * 4);
        } else {
            int kf, vf;
            orc_kv_mode_formats(mode, &kf, &vf);
            orc_kv_dequant(kf, kq, ek, (int64_t)start_pos * kvd);
            orc_kv_dequant(vf, vq, ev, (int64_t)start_pos * kvd);
        }
        if (pre_rope && rkc) orc_rope_neox(ek, rkc, rks, start_pos, Hkv, dh, 0);
    }
    memcpy(ek + (size_t)start_pos * kvd, kcur, (size_t)T * kvd * 4);
    memcpy(ev + (size_t)start_pos * kvd, vcur, (size_t)T * kvd * 4);
    int rep = H / Hkv;
    gqa_head_job jobs[64];
    pthread_t th[64];
    int nw = nt < 1 ? 1 : nt > H ? H : nt > 64 ? 64 : nt;
    for (int w = 0; w < nw; w++) {
        jobs[w] = (gqa_head_job){q, ek, ev, out, H, rep, dh, kvd, start_pos, T, w, nw};
        if (w) pthread_create(&th[w], NULL, gqa_head_worker, &jobs[w]);
    }
    gqa_head_worker(&jobs[0]);
    for (int w = 1; w < nw; w++) pthread_join(th[w], NULL);
    free(ek);
    free(ev);
}

/* ------------------------------------------------------------------ */
/* GQA model (infer/infer_gqa.cpp + arch/gqa/gqa_layer.cu)              */
/* ------------------------------------------------------------------ */

struct orc_gqa {
    orc_gqa_cfg c;
    orc_gqa_layer_w* layers;
    int kf, vf, kbb, vbb;
    size_t bpl;                 /* blocks per layer */
    uint8_t* qcache;            /* [L][K blocks][V blocks] */
    float* fcache;              /* [L][2][max_seq][kvd] */
    float* last_kv;             /* [L][2][cap][kvd] fp32 K/V of the last call */
    int last_cap;
};

orc_gqa* orc_gqa_create(const orc_gqa_cfg* cfg) {
    orc_gqa* m = (orc_gqa*)calloc(1, sizeof(orc_gqa));
    m->c = *cfg;
    m->layers = (orc_gqa_layer_w*)malloc(sizeof(orc_gqa_layer_w) * cfg->n_layers);
    memcpy(m->layers, cfg->layers, sizeof(orc_gqa_layer_w) * cfg->n_layers);
    m->c.layers = m->layers;
    int kvd = cfg->n_kv_heads * cfg->head_dim;
    if (cfg->kv_mode > 0) {
        orc_kv_mode_formats(cfg->kv_mode, &m->kf, &m->vf);
        m->kbb = orc_kv_block_bytes(m->kf);
        m->vbb = orc_kv_block_bytes(m->vf);
        m->bpl = (size_t)cfg->max_seq * kvd / 32;
        m->qcache = (uint8_t*)calloc((size_t)cfg->n_layers * m->bpl * (m->kbb + m->vbb), 1);
    } else {
        m->fcache = (float*)calloc((size_t)cfg->n_layers * 2 * cfg->max_seq * kvd, 4);
    }
    return m;
}

void orc_gqa_destroy(orc_gqa* m) {
    if (!m) return;
    free(m->layers); free(m->qcache); free(m->fcache); free(m->last_kv);
    free(m);
}

void* orc_gqa_cache(orc_gqa* m, int layer, int which_v, size_t* bytes) {
    int kvd = m->c.n_kv_heads * m->c.head_dim;
    if (m->c.kv_mode > 0) {
        uint8_t* base = m->qcache + (size_t)layer * m->bpl * (m->kbb + m->vbb);
        if (bytes) *bytes = m->bpl * (which_v ? m->vbb : m->kbb);
        return which_v ? base + m->bpl * m->kbb : base;
    }
    if (bytes) *bytes = (size_t)m->c.max_seq * kvd * 4;
    return m->fcache + ((size_t)layer * 2 + (which_v ? 1 : 0)) * m->c.max_seq * kvd;
}

const float* orc_gqa_last_kv(orc_gqa* m, int layer, int which_v) {
    int kvd = m->c.n_kv_heads * m->c.head_dim;
    if (!m->last_kv) return NULL;
    return m->last_kv + ((size_t)layer * 2 + (which_v ? 1 : 0)) * m->last_cap * kvd;
}

static void norm_rows(const orc_gqa_cfg* c, float* x, const float* w, int n) {
    if (c->use_rms_norm) orc_rms_norm(x, w, n, c->dim, 1e-5f);
    else orc_layer_norm(x, w, n, c->dim, 1e-5f);
}

int orc_gqa_forward(orc_gqa* m, const int* ids, int T, int start_pos, float* logits, int last_only) {
    const orc_gqa_cfg* c = &m->c;
    int d = c->dim, H = c->n_heads, Hkv = c->n_kv_heads, dh = c->head_dim, hd = c->hidden;
    int kvd = Hkv * dh, nt = c->nthreads;
    if (start_pos + T > c->max_seq) return -3;
    float* h = (float*)malloc((size_t)T * d * 4);
    float* a = (float*)malloc((size_t)T * (d > H * dh ? d : H * dh) * 4);
    float* q = (float*)malloc((size_t)T * H * dh * 4);
    float* k = (float*)malloc((size_t)T * kvd * 4);
    float* v = (float*)malloc((size_t)T * kvd * 4);
    float* kraw = (float*)malloc((size_t)T * kvd * 4);
    float* att = (float*)malloc((size_t)T * H * dh * 4);
    float* g = (float*)malloc((size_t)T * hd * 4);
    float* u = (float*)malloc((size_t)T * hd * 4);
    if (m->last_cap < T) {
        free(m->last_kv);
        m->last_kv = (float*)malloc((size_t)c->n_layers * 2 * T * kvd * 4);
        m->last_cap = T;
    }
    orc_embedding(c->wte, c->qt_wte, ids, h, T, d);
    for (int l = 0; l < c->n_layers; l++) {
        const orc_gqa_layer_w* L = &c->layers[l];
        memcpy(a, h, (size_t)T * d * 4);
        norm_rows(c, a, L->ln1, T);
        orc_linear(L->w_q, L->qt_q, a, q, T, H * dh, d, nt);
        orc_linear(L->w_k, L->qt_k, a, k, T, kvd, d, nt);
        orc_linear(L->w_v, L->qt_v, a, v, T, kvd, d, nt);
        if (c->pre_rope) memcpy(kraw, k, (size_t)T * kvd * 4);
        if (L->rope_q_cos) orc_rope_neox(q, L->rope_q_cos, L->rope_q_sin, T, H, dh, start_pos);
        if (L->rope_k_cos) orc_rope_neox(k, L->rope_k_cos, L->rope_k_sin, T, Hkv, dh, start_pos);
        const float* kc = c->pre_rope ? kraw : k;
        memcpy(m->last_kv + ((size_t)l * 2) * m->last_cap * kvd, kc, (size_t)T * kvd * 4);
        memcpy(m->last_kv + ((size_t)l * 2 + 1) * m->last_cap * kvd, v, (size_t)T * kvd * 4);
        /* append (gqa_layer.cu:155-190) */
        if (c->kv_mode > 0) {
            uint8_t* ck = (uint8_t*)orc_gqa_cache(m, l, 0, NULL);
            uint8_t* cv = (uint8_t*)orc_gqa_cache(m, l, 1, NULL);
            size_t off = (size_t)start_pos * kvd / 32;
            orc_kv_quantize(m->kf, kc, ck + off * m->kbb, (int64_t)T * kvd);
            orc_kv_quantize(m->vf, v, cv + off * m->vbb, (int64_t)T * kvd);
            gqa_attention_nt(q, k, v, NULL, NULL, ck, cv, c->kv_mode, c->pre_rope,
                             L->rope_k_cos, L->rope_k_sin, T, start_pos, H, Hkv, dh, att, nt > 0 ? nt : orc_num_threads());
        } else {
            float* ck = (float*)orc_gqa_cache(m, l, 0, NULL);
            float* cv = (float*)orc_gqa_cache(m, l, 1, NULL);
            memcpy(ck + (size_t)start_pos * kvd, kc, (size_t)T * kvd * 4);
            memcpy(cv + (size_t)start_pos * kvd, v, (size_t)T * kvd * 4);
            gqa_attention_nt(q, k, v, ck, cv, NULL, NULL, 0, c->pre_rope,
                             L->rope_k_cos, L->rope_k_sin, T, start_pos, H, Hkv, dh, att, nt > 0 ? nt : orc_num_threads());
        }
        orc_linear(L->w_o, L->qt_o, att, a, T, d, H * dh, nt);   /* out of place */
        orc_add(h, h, a, T * d);
        memcpy(a, h, (size_t)T * d * 4);
        norm_rows(c, a, L->ln2, T);
        orc_linear(L->w1, L->qt_1, a, g, T, hd, d, nt);
        orc_linear(L->w3, L->qt_3, a, u, T, hd, d, nt);
        orc_silu_mul(g, g, u, T * hd);
        orc_linear(L->w2, L->qt_2, g, a, T, d, hd, nt);
        orc_add(h, h, a, T * d);
    }
    if (c->ln_f) norm_rows(c, h, c->ln_f, T);
    const void* lm = c->lm_head ? c->lm_head : c->wte;
    int qlm = c->lm_head ? c->qt_lm : c->qt_wte;
    if (last_only) orc_linear(lm, qlm, h + (size_t)(T - 1) * d, logits, 1, c->vocab, d, nt);
    else orc_linear(lm, qlm, h, logits, T, c->vocab, d, nt);
    free(h); free(a); free(q); free(k); free(v); free(kraw); free(att); free(g); free(u);
    return 0;
}

int orc_gqa_generate(orc_gqa* m, const int* prompt, int n_prompt, int steps, int* out_ids) {
    int V = m->c.vocab;
    int* gen = (int*)malloc(sizeof(int) * (n_prompt + steps));
    memcpy(gen, prompt, sizeof(int) * n_prompt);
    float* logits = (float*)malloc((size_t)V * 4);
    int len = n_prompt, rc = 0;
    for (int step = 0; step < steps; step++) {
        int T = step == 0 ? len : 1;
        int sp = step == 0 ? 0 : len - 1;
        rc = orc_gqa_forward(m, gen + sp, T, sp, logits, 1);
        if (rc) break;
        int nx = orc_argmax(logits, V);
        gen[len++] = nx;
        out_ids[step] = nx;
    }
    free(gen);
    free(logits);
    return rc;
}

/* ------------------------------------------------------------------ */
/* DeepSeek MLA + MoE (arch/mla/deepseek_mla_layer.cu, infer_mla.cpp)   */
/* ------------------------------------------------------------------ */

/* deepseek_mla_layer.cu:310-326 generalized to E experts, top k */
void orc_moe_topk(const float* lp, int E, int k, int* topk, float* topw) {
    float max_lp = lp[0];
    for (int e = 1; e < E; e++) if (lp[e] > max_lp) max_lp = lp[e];   /* std::max_element */
    float sum_exp = 0.0f;
    for (int e = 0; e < E; e++) sum_exp += expf(lp[e] - max_lp);
    float inv_sum = 1.0f / sum_exp;
    for (int j = 0; j < k; j++) { topk[j] = -1; topw[j] = -1e10f; }
    for (int e = 0; e < E; e++) {
        float w = expf(lp[e] - max_lp) * inv_sum;
        if (w > topw[0]) {
            topw[0] = w; topk[0] = e;
            for (int j = 0; j < k - 1 && topw[j] > topw[j + 1]; j++) {
                float tw = topw[j]; topw[j] = topw[j + 1]; topw[j + 1] = tw;
                int ti = topk[j]; topk[j] = topk[j + 1]; topk[j + 1] = ti;
            }
        }
    }
}

struct orc_mla {
    orc_mla_cfg c;
    orc_mla_layer_w* layers;
    float* cache;      /* [L][max_seq*(rope + H*nope + H*v)] */
    size_t per_layer;
    float* latent_tap; /* optional [L][max_seq][dc + rope]: records of the rows forward() stores */
};

void orc_mla_set_latent_tap(orc_mla* m, float* tap) { m->latent_tap = tap; }

orc_mla* orc_mla_create(const orc_mla_cfg* cfg) {
    orc_mla* m = (orc_mla*)calloc(1, sizeof(orc_mla));
    m->c = *cfg;
    m->layers = (orc_mla_layer_w*)malloc(sizeof(orc_mla_layer_w) * cfg->n_layers);
    memcpy(m->layers, cfg->layers, sizeof(orc_mla_layer_w) * cfg->n_layers);
    m->c.layers = m->layers;
    int H = cfg->n_heads;
    m->per_layer = (size_t)cfg->max_seq * (cfg->rope + (size_t)H * cfg->nope + (size_t)H * cfg->v_dim);
    m->cache = (float*)calloc((size_t)cfg->n_layers * m->per_layer, 4);
    return m;
}

void orc_mla_destroy(orc_mla* m) {
    if (!m) return;
    free(m->layers); free(m->cache);
    free(m);
}

const float* orc_mla_cache(orc_mla* m, int layer, int which) {
    const orc_mla_cfg* c = &m->c;
    float* base = m->cache + (size_t)layer * m->per_layer;
    if (which == 0) return base;
    base += (size_t)c->max_seq * c->rope;
    if (which == 1) return base;
    return base + (size_t)c->max_seq * c->n_heads * c->nope;
}

/* Positions 0..n_pos-1 of one layer's cache from latent records
 * [c (dc) | k_pe (rope)] (the c of a record is RMSNorm(c_kv)*k_norm, the
 * k_pe is already rotated): the same rows orc_mla_forward stores for those
 * positions (deepseek_mla_layer.cu:196,221-228): k_pe as is, and
 * [K_nope | V] = W_kv_b c through orc_linear. */
int orc_mla_load_latent(orc_mla* m, int layer, const float* rec, int n_pos) {
    const orc_mla_cfg* c = &m->c;
    if (layer < 0 || layer >= c->n_layers || n_pos < 0 || n_pos > c->max_seq) return -3;
    const int H = c->n_heads, nope = c->nope, rope = c->rope, vd = c->v_dim, dc = c->dc, R = dc + rope;
    const orc_mla_layer_w* L = &c->layers[layer];
    if (!n_pos) return 0;
    float* Cn = (float*)malloc((size_t)n_pos * dc * 4);
    float* KVB = (float*)malloc((size_t)n_pos * H * (nope + vd) * 4);
    for (int p = 0; p < n_pos; p++) memcpy(Cn + (size_t)p * dc, rec + (size_t)p * R, (size_t)dc * 4);
    int rc = orc_linear(L->w_kv_b, L->qt_kv_b, Cn, KVB, n_pos, H * (nope + vd), dc, c->nthreads);
    float* kpe_c = (float*)orc_mla_cache(m, layer, 0);
    float* kn_c = (float*)orc_mla_cache(m, layer, 1);
    float* v_c = (float*)orc_mla_cache(m, layer, 2);
    for (int p = 0; p < n_pos && !rc; p++) {
        memcpy(kpe_c + (size_t)p * rope, rec + (size_t)p * R + dc, (size_t)rope * 4);
        memcpy(kn_c + (size_t)p * H * nope, KVB + (size_t)p * H * (nope + vd), (size_t)H * nope * 4);
        memcpy(v_c + (size_t)p * H * vd, KVB + (size_t)p * H * (nope + vd) + (size_t)H * nope, (size_t)H * vd * 4);
    }
    free(Cn);
    free(KVB);
    return rc;
}

/* SwiGLU block: out[d] = W_down(silu(W_gate x) * (W_up x)) */
static void swiglu_rows(const void* wg, const void* wu, int qt_gu, const void* wd, int qt_d,
                        const float* x, float* out, int T, int d, int hid, int nt) {
    float* g = (float*)malloc((size_t)T * hid * 4);
    float* u = (float*)malloc((size_t)T * hid * 4);
    orc_linear(wg, qt_gu, x, g, T, hid, d, nt);
    orc_linear(wu, qt_gu, x, u, T, hid, d, nt);
    orc_silu_mul(g, g, u, T * hid);
    orc_linear(wd, qt_d, g, out, T, d, hid, nt);
    free(g); free(u);
}

typedef struct {
    const float *Q, *kn_c, *kpe_c, *v_c;
    float* att;
    int H, nope, rope, vd, T, start_pos, w, nw;
    float *Kh, *Vh;    /* NULL: the worker allocates its own */
    int ms;
} mla_head_job;

/* heads w, w + nw, ... of one layer's attention (orc_mla_forward) */
static void* mla_head_worker(void* arg) {
    mla_head_job* j = (mla_head_job*)arg;
    const int H = j->H, nope = j->nope, rope = j->rope, vd = j->vd, dq = nope + rope;
    float* Kh = j->Kh ? j->Kh : (float*)malloc((size_t)j->ms * dq * 4);
    float* Vh = j->Vh ? j->Vh : (float*)malloc((size_t)j->ms * vd * 4);
    float qv[1024];
    const int last = j->start_pos + j->T;
    for (int hh = j->w; hh < H; hh += j->nw) {
        for (int p = 0; p < last; p++) {
            memcpy(Kh + (size_t)p * dq, j->kn_c + (size_t)p * H * nope + (size_t)hh * nope, (size_t)nope * 4);
            memcpy(Kh + (size_t)p * dq + nope, j->kpe_c + (size_t)p * rope, (size_t)rope * 4);
            memcpy(Vh + (size_t)p * vd, j->v_c + (size_t)p * H * vd + (size_t)hh * vd, (size_t)vd * 4);
        }
        for (int t = 0; t < j->T; t++) {
            const float* qrow = j->Q + (size_t)t * H * dq;
            memcpy(qv, qrow + (size_t)hh * nope, (size_t)nope * 4);
            memcpy(qv + nope, qrow + (size_t)H * nope + (size_t)hh * rope, (size_t)rope * 4);
            orc_attn_rows(qv, dq, Kh, dq, Vh, vd, j->att + (size_t)t * H * vd + (size_t)hh * vd, vd,
                          j->start_pos + t, 1, dq, vd);
        }
    }
    if (!j->Kh) free(Kh);
    if (!j->Vh) free(Vh);
    return NULL;
}

int orc_mla_forward(orc_mla* m, const int* ids, int T, int start_pos, float* logits, int last_only) {
    const orc_mla_cfg* c = &m->c;
    const int d = c->dim, H = c->n_heads, nope = c->nope, rope = c->rope, vd = c->v_dim, dc = c->dc;
    const int dq = nope + rope, nt = c->nthreads, ms = c->max_seq;
    if (start_pos < 0 || start_pos + T > ms) return -3;
    float* h = (float*)malloc((size_t)T * d * 4);
    float* a = (float*)malloc((size_t)T * d * 4);
    float* Q = (float*)malloc((size_t)T * H * dq * 4);
    float* KVA = (float*)malloc((size_t)T * (dc + rope) * 4);
    float* Cn = (float*)malloc((size_t)T * dc * 4);
    float* KVB = (float*)malloc((size_t)T * H * (nope + vd) * 4);
    float* att = (float*)malloc((size_t)T * H * vd * 4);
    float* tmp = (float*)malloc((size_t)T * d * 4);
    float* Kh = (float*)malloc((size_t)ms * dq * 4);
    float* Vh = (float*)malloc((size_t)ms * vd * 4);
    orc_embedding(c->wte, c->qt_wte, ids, h, T, d);
    for (int l = 0; l < c->n_layers; l++) {
        const orc_mla_layer_w* L = &c->layers[l];
        float* kpe_c = (float*)orc_mla_cache(m, l, 0);
        float* kn_c = (float*)orc_mla_cache(m, l, 1);
        float* v_c = (float*)orc_mla_cache(m, l, 2);
        memcpy(a, h, (size_t)T * d * 4);
        orc_rms_norm(a, L->ln1, T, d, 1e-5f);                                  /* :180-181 */
        orc_linear(L->w_q, L->qt_q, a, Q, T, H * dq, d, nt);                  /* :184 */
        orc_linear(L->w_kv_a, L->qt_kv_a, a, KVA, T, dc + rope, d, nt);       /* :187 */
        for (int t = 0; t < T; t++) memcpy(Cn + (size_t)t * dc, KVA + (size_t)t * (dc + rope), (size_t)dc * 4);
        orc_rms_norm(Cn, L->k_norm, T, dc, 1e-5f);                             /* :192 */
        orc_linear(L->w_kv_b, L->qt_kv_b, Cn, KVB, T, H * (nope + vd), dc, nt);  /* :196 */
        for (int t = 0; t < T; t++) {
            const int pos = start_pos + t;
            float* qr = Q + (size_t)t * H * dq + (size_t)H * nope;             /* [H*rope] of this row */
            float* kpe = KVA + (size_t)t * (dc + rope) + dc;
            if (L->rope_cos) {                                                 /* :202-203 */
                orc_rope_neox(qr, L->rope_cos, L->rope_sin, 1, H, rope, pos);
                orc_rope_neox(kpe, L->rope_cos, L->rope_sin, 1, 1, rope, pos);
            }
            memcpy(kpe_c + (size_t)pos * rope, kpe, (size_t)rope * 4);
            if (m->latent_tap) {
                float* r = m->latent_tap + ((size_t)l * ms + pos) * (dc + rope);
                memcpy(r, Cn + (size_t)t * dc, (size_t)dc * 4);
                memcpy(r + dc, kpe, (size_t)rope * 4);
            }
            memcpy(kn_c + (size_t)pos * H * nope, KVB + (size_t)t * H * (nope + vd), (size_t)H * nope * 4);
            memcpy(v_c + (size_t)pos * H * vd, KVB + (size_t)t * H * (nope + vd) + (size_t)H * nope,
                   (size_t)H * vd * 4);
        }
        /* attention per head over keys 0..pos: K = [K_nope | k_pe], V, scale
         * rsqrt(dq); heads are independent and run on the worker threads */
        {
            mla_head_job jobs[64];
            pthread_t th[64];
            int nth = nt > 0 ? nt : orc_num_threads();
            if (nth > H) nth = H;
            if (nth > 64) nth = 64;
            for (int w = 0; w < nth; w++) {
                jobs[w] = (mla_head_job){Q, kn_c, kpe_c, v_c, att, H, nope, rope, vd, T, start_pos, w, nth,
                                         w == 0 ? Kh : NULL, w == 0 ? Vh : NULL, ms};
                if (w) pthread_create(&th[w], NULL, mla_head_worker, &jobs[w]);
            }
            mla_head_worker(&jobs[0]);
            for (int w = 1; w < nth; w++) pthread_join(th[w], NULL);
        }
        orc_linear(L->w_o, L->qt_o, att, tmp, T, d, H * vd, nt);               /* :271 (out of place) */
        orc_add(h, h, tmp, T * d);
        memcpy(a, h, (size_t)T * d * 4);
        orc_rms_norm(a, L->ln2, T, d, 1e-5f);                                  /* :276 */
        if (!L->is_moe) {
            swiglu_rows(L->w1, L->w3, L->qt_1, L->w2, L->qt_2, a, tmp, T, d, L->hidden, nt);   /* :281-286 */
            orc_add(h, h, tmp, T * d);
            continue;
        }
        /* forward_moe (:291-350), per token */
        const int E = c->n_experts, K = c->top_k, F = c->expert_ffn;
        float* lg = (float*)malloc((size_t)E * 4);
        float* acc = (float*)malloc((size_t)d * 4);
        float* eo = (float*)malloc((size_t)d * 4);
        int topk[64];
        float topw[64];
        for (int t = 0; t < T; t++) {
            const float* at = a + (size_t)t * d;
            swiglu_rows(L->gate_sh, L->up_sh, L->qt_sh_gu, L->down_sh, L->qt_sh_dn, at, acc, 1, d,
                        L->shared_hidden, nt);                                 /* :297-302 */
            orc_linear(L->gate_inp, L->qt_gate_inp, at, lg, 1, E, d, nt);      /* :305 */
            orc_moe_topk(lg, E, K, topk, topw);
            for (int j = 0; j < K; j++) {
                const int e = topk[j];
                if (e < 0) continue;
                swiglu_rows((const uint8_t*)L->gate_exps + (int64_t)e * L->stride_gu,
                            (const uint8_t*)L->up_exps + (int64_t)e * L->stride_gu, L->qt_gu,
                            (const uint8_t*)L->down_exps + (int64_t)e * L->stride_dn, L->qt_dn, at, eo, 1, d, F,
                            nt);                                               /* :332-343 */
                orc_saxpy(acc, eo, topw[j], d);                                /* :345 */
            }
            orc_add(h + (size_t)t * d, h + (size_t)t * d, acc, d);            /* :349 */
        }
        free(lg); free(acc); free(eo);
    }
    if (c->ln_f) orc_rms_norm(h, c->ln_f, T, d, 1e-5f);
    const void* lm = c->lm_head ? c->lm_head : c->wte;
    int qlm = c->lm_head ? c->qt_lm : c->qt_wte;
    if (last_only) orc_linear(lm, qlm, h + (size_t)(T - 1) * d, logits, 1, c->vocab, d, nt);
    else orc_linear(lm, qlm, h, logits, T, c->vocab, d, nt);
    free(h); free(a); free(Q); free(KVA); free(Cn); free(KVB); free(att); free(tmp); free(Kh); free(Vh);
    return 0;
}

int orc_mla_generate(orc_mla* m, const int* prompt, int n_prompt, int steps, int* out_ids) {
    int V = m->c.vocab;
    int* gen = (int*)malloc(sizeof(int) * (n_prompt + steps));
    memcpy(gen, prompt, sizeof(int) * n_prompt);
    float* logits = (float*)malloc((size_t)V * 4);
    int len = n_prompt, rc = 0;
    for (int step = 0; step < steps; step++) {
        int T = step == 0 ? len : 1;
        int sp = step == 0 ? 0 : len - 1;
        rc = orc_mla_forward(m, gen + sp, T, sp, logits, 1);
        if (rc) break;
        int nx = orc_argmax(logits, V);
        gen[len++] = nx;
        out_ids[step] = nx;
    }
    free(gen);
    free(logits);
    return rc;
}

/* ------------------------------------------------------------------ */
/* RINA Jamba hybrid (rina_ssm_layer.cu, rina_mla_layer.cu)            */
/* ------------------------------------------------------------------ */

struct orc_jamba {
    orc_jamba_cfg c;
    orc_jamba_layer_w* layers;
    float** lcs;     /* SSM layers: [H*dh] log cumulative decay (one per scan thread) */
    float** wcs;     /* SSM layers: [H*dh] weighted cumulative memory */
    float** kc;      /* RMLA layers: [max_seq][Hkv*(dh+dhr)] */
    float** vc;      /* RMLA layers: [max_seq][Hkv*dh] */
    uint8_t** kq;    /* rmla_kv_mode q2k_q1v: key content q2_1 [max_seq][Hkv][dh/32] blocks */
    uint8_t** vq;    /* rmla_kv_mode q2k_q1v: value q1_0 [max_seq][Hkv][dh/32] records */
};

const float* orc_jamba_fp32_cache(orc_jamba* m, int layer, int which) {
    if (layer < 0 || layer >= m->c.n_layers || m->layers[layer].type == ORC_JAMBA_SSM) return NULL;
    return which ? m->vc[layer] : m->kc[layer];
}

const uint8_t* orc_jamba_packed_cache(orc_jamba* m, int layer, int part) {
    if (layer < 0 || layer >= m->c.n_layers || m->c.rmla_kv_mode != ORC_KV_Q2K_Q1V || !m->kq) return NULL;
    return part == 0 ? m->kq[layer] : part == 1 ? m->vq[layer] : NULL;
}

orc_jamba* orc_jamba_create(const orc_jamba_cfg* cfg) {
    orc_jamba* m = (orc_jamba*)calloc(1, sizeof(orc_jamba));
    m->c = *cfg;
    int L = cfg->n_layers;
    m->layers = (orc_jamba_layer_w*)malloc(sizeof(orc_jamba_layer_w) * L);
    memcpy(m->layers, cfg->layers, sizeof(orc_jamba_layer_w) * L);
    m->c.layers = m->layers;
    m->lcs = (float**)calloc(L, sizeof(float*));
    m->wcs = (float**)calloc(L, sizeof(float*));
    m->kc = (float**)calloc(L, sizeof(float*));
    m->vc = (float**)calloc(L, sizeof(float*));
    const int H = cfg->n_heads, Hkv = cfg->n_kv_heads, dh = cfg->head_dim, dhr = cfg->dhr;
    for (int l = 0; l < L; l++) {
        if (m->layers[l].type == ORC_JAMBA_SSM) {
            m->lcs[l] = (float*)calloc((size_t)H * dh, 4);
            m->wcs[l] = (float*)calloc((size_t)H * dh, 4);
        } else {
            m->kc[l] = (float*)calloc((size_t)cfg->max_seq * Hkv * (dh + dhr), 4);
            m->vc[l] = (float*)calloc((size_t)cfg->max_seq * Hkv * dh, 4);
        }
    }
    if (cfg->rmla_kv_mode == ORC_KV_Q2K_Q1V) {
        m->kq = (uint8_t**)calloc(L, sizeof(uint8_t*));
        m->vq = (uint8_t**)calloc(L, sizeof(uint8_t*));
        for (int l = 0; l < L; l++)
            if (m->layers[l].type != ORC_JAMBA_SSM) {
                m->kq[l] = (uint8_t*)calloc((size_t)cfg->max_seq * Hkv * (dh / 32), 10);
                m->vq[l] = (uint8_t*)calloc((size_t)cfg->max_seq * Hkv * (dh / 32), 6);
            }
    }
    return m;
}

void orc_jamba_destroy(orc_jamba* m) {
    if (!m) return;
    for (int l = 0; l < m->c.n_layers; l++) {
        free(m->lcs[l]); free(m->wcs[l]); free(m->kc[l]); free(m->vc[l]);
        if (m->kq) { free(m->kq[l]); free(m->vq[l]); }
    }
    free(m->lcs); free(m->wcs); free(m->kc); free(m->vc); free(m->kq); free(m->vq); free(m->layers);
    free(m);
}

static float orc_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }   /* ssm_kernels_fp32.cu:6-8 */

/* one SSM layer on token rows [T, d] (rina_ssm_layer.cu:90-126) */
static void jamba_ssm(orc_jamba* m, int l, float* h, int T) {
    const orc_jamba_cfg* c = &m->c;
    const orc_jamba_layer_w* L = &c->layers[l];
    const int d = c->dim, H = c->n_heads, dh = c->head_dim, dc = c->dc, S = c->ssm_steps, nt = c->nthreads;
    const int d2 = d + H * dh;
    float* x2 = (float*)malloc((size_t)T * d2 * 4);
    float* a = (float*)malloc((size_t)T * d * 4);
    float* cq = (float*)malloc((size_t)T * dc * 4);
    float* mem = (float*)malloc((size_t)3 * T * H * dh * 4);
    float* dec = (float*)malloc((size_t)3 * T * H * 4);
    float* tmp = (float*)malloc((size_t)T * d * 4);
    memcpy(a, h, (size_t)T * d * 4);
    orc_layer_norm(a, L->ln1, T, d, 1e-5f);                                    /* :93-95 */
    orc_linear(L->w_dq, L->qt, a, cq, T, dc, d, nt);                            /* :96 */
    orc_layer_norm(cq, L->q_norm, T, dc, 1e-5f);                                /* :97 */
    for (int k = 0; k < 3; k++) {
        if (k < S) {
            orc_linear(L->w_mem[k], L->qt, cq, mem + (size_t)k * T * H * dh, T, H * dh, dc, nt);   /* :100 */
            orc_linear(L->w_decay[k], L->qt, cq, dec + (size_t)k * T * H, T, H, dc, nt);           /* :101 */
            for (int i = 0; i < T * H; i++) dec[(size_t)k * T * H + i] = orc_sigmoid(dec[(size_t)k * T * H + i]);
        } else {   /* fewer steps: neutral factors */
            memset(mem + (size_t)k * T * H * dh, 0, (size_t)T * H * dh * 4);
            for (int i = 0; i < T * H; i++) dec[(size_t)k * T * H + i] = 1.0f;
        }
    }
    /* ssm_agg (ssm_kernels_fp32.cu:14-22) then ssm_scan (:30-42), per (h, d) thread over t */
    for (int t = 0; t < T; t++) {
        for (int hh = 0; hh < H; hh++) {
            const size_t i = (size_t)t * H + hh;
            const float dd0 = dec[i], dd1 = dec[(size_t)T * H + i], dd2 = dec[(size_t)2 * T * H + i];
            float da = dd0 * dd1 * dd2;
            if (da <= 1e-38f) da = 1e-38f;
            for (int dd = 0; dd < dh; dd++) {
                const size_t j = i * dh + dd;
                const float m0 = mem[j], m1 = mem[(size_t)T * H * dh + j], m2 = mem[(size_t)2 * T * H * dh + j];
                const float ma = fmaf(m0 * dd1, dd2, m1 * dd2) + m2;
                float* lcs = &m->lcs[l][hh * dh + dd];
                float* wcs = &m->wcs[l][hh * dh + dd];
                *lcs += logf(da);
                const float ca = expf(*lcs);
                *wcs += ma / fmaxf(ca, 1e-30f);
                x2[(size_t)t * d2 + d + hh * dh + dd] = ca * *wcs;
            }
        }
        memcpy(x2 + (size_t)t * d2, a + (size_t)t * d, (size_t)d * 4);          /* :110-113 [x_ln | sf] */
    }
    orc_linear(L->w_out, L->qt, x2, tmp, T, d, d2, nt);                         /* :114 */
    orc_add(h, h, tmp, T * d);
    free(x2); free(a); free(cq); free(mem); free(dec); free(tmp);
}

/* HF RoPE pairs (2i, 2i+1) of one head row at position pos (ops/rope.cu:212-227) */
static void rope_hf_row(float* row, const float* ct, const float* st, int d, int pos) {
    const int half = d / 2;
    for (int i = 0; i < half; i++) {
        const float cc = ct[(int64_t)pos * half + i], ss = st[(int64_t)pos * half + i];
        const float x0 = row[2 * i], x1 = row[2 * i + 1];
        row[2 * i] = fmaf(x0, cc, -(x1 * ss));
        row[2 * i + 1] = fmaf(x0, ss, x1 * cc);
    }
}

/* one RINA-MLA layer on token rows [T, d] at positions start_pos.. (rina_mla_layer.cu:65-98) */
typedef struct {
    const float *q, *qr, *kc, *vc;
    const float *kcur, *vcur;   /* packed cache: this call's fp32 rows [T][Hkv*dq], [T][Hkv*dh] (else NULL) */
    float* att;
    int H, Hkv, dh, dhr, T, start_pos, w, nw;
} rmla_rows_job;

/* query rows t = w, w + nw, ... of the RINA-MLA attention: every head of
 * the row over keys 0..start_pos + t (flash_fp32 semantics).  With kcur set
 * (packed cache) kc / vc hold every row of the call dequantized; the worker
 * reads them through a private copy in which row start_pos + t holds its
 * fp32 values while that row attends, so each row sees the earlier rows
 * through their packs and itself in fp32, as a row-by-row append would. */
static void* rmla_rows_worker(void* arg) {
    rmla_rows_job* j = (rmla_rows_job*)arg;
    const int H = j->H, Hkv = j->Hkv, dh = j->dh, dhr = j->dhr, dq = dh + dhr, rep = H / Hkv;
    const size_t kr = (size_t)Hkv * dq, vr = (size_t)Hkv * dh, rows = (size_t)j->start_pos + j->T;
    const float *kc = j->kc, *vc = j->vc;
    float *kp = NULL, *vp = NULL;
    if (j->kcur) {
        kp = (float*)malloc(rows * kr * 4);
        vp = (float*)malloc(rows * vr * 4);
        memcpy(kp, j->kc, rows * kr * 4);
        memcpy(vp, j->vc, rows * vr * 4);
        kc = kp;
        vc = vp;
    }
    float qv[512];
    for (int t = j->w; t < j->T; t += j->nw) {
        const size_t pos = (size_t)j->start_pos + t;
        if (kp) {
            memcpy(kp + pos * kr, j->kcur + (size_t)t * kr, kr * 4);
            memcpy(vp + pos * vr, j->vcur + (size_t)t * vr, vr * 4);
        }
        for (int hh = 0; hh < H; hh++) {
            const int kv = hh / rep;
            memcpy(qv, j->q + ((size_t)t * H + hh) * dh, (size_t)dh * 4);
            memcpy(qv + dh, j->qr + ((size_t)t * H + hh) * dhr, (size_t)dhr * 4);
            orc_attn_rows(qv, dq, kc + (size_t)kv * dq, Hkv * dq, vc + (size_t)kv * dh, Hkv * dh,
                          j->att + ((size_t)t * H + hh) * dh, dh, (int)pos, 1, dq, dh);
        }
        if (kp) {
            memcpy(kp + pos * kr, j->kc + pos * kr, kr * 4);
            memcpy(vp + pos * vr, j->vc + pos * vr, vr * 4);
        }
    }
    free(kp);
    free(vp);
    return NULL;
}

static void jamba_rmla(orc_jamba* m, int l, float* h, int T, int start_pos) {
    const orc_jamba_cfg* c = &m->c;
    const orc_jamba_layer_w* L = &c->layers[l];
    const int d = c->dim, H = c->n_heads, Hkv = c->n_kv_heads, dh = c->head_dim, dhr = c->dhr, dc = c->dc;
    const int dq = dh + dhr, nt = c->nthreads;
    float* a = (float*)malloc((size_t)T * d * 4);
    float* cq = (float*)malloc((size_t)T * dc * 4);
    float* q = (float*)malloc((size_t)T * H * dh * 4);
    float* k = (float*)malloc((size_t)T * Hkv * dh * 4);
    float* v = (float*)malloc((size_t)T * Hkv * dh * 4);
    float* qr = (float*)malloc((size_t)T * H * dhr * 4);
    float* kr = (float*)malloc((size_t)T * Hkv * dhr * 4);
    float* att = (float*)malloc((size_t)T * H * dh * 4);
    float* tmp = (float*)malloc((size_t)T * d * 4);
    memcpy(a, h, (size_t)T * d * 4);
    orc_layer_norm(a, L->ln1, T, d, 1e-5f);                                    /* :70 */
    orc_linear(L->w_dq, L->qt, a, cq, T, dc, d, nt);                            /* :72 w_dqkv */
    orc_layer_norm(cq, L->q_norm, T, dc, 1e-5f);                                /* :73 */
    orc_linear(L->w_uq, L->qt, cq, q, T, H * dh, dc, nt);                       /* :75 */
    orc_linear(L->w_uk, L->qt, cq, k, T, Hkv * dh, dc, nt);                     /* :76 */
    orc_linear(L->w_k2v, L->qt, k, v, T, Hkv * dh, Hkv * dh, nt);               /* :77 */
    orc_linear(L->w_qr, L->qt, a, qr, T, H * dhr, d, nt);                       /* :78 */
    orc_linear(L->w_kr, L->qt, a, kr, T, Hkv * dhr, d, nt);                     /* :79 */
    /* q2k_q1v cache: position p attends to positions < p through the packed
     * cache (key content and values dequantized; the RoPE part is kept fp32)
     * and to itself through its fp32 rows, as the GQA composition reads its
     * quantized cache (gqa_layer.cu:203-245).  A T-row call equals T
     * single-row calls: every row is packed on append (kernels/quantize.cu:
     * 74-185) and stored dequantized, and each query row reads its own
     * position's fp32 values (rmla_rows_worker). */
    const int qkv = c->rmla_kv_mode == ORC_KV_Q2K_Q1V;
    float* kcur = qkv ? (float*)malloc((size_t)T * Hkv * dq * 4) : NULL;
    float* vcur = qkv ? (float*)malloc((size_t)T * Hkv * dh * 4) : NULL;
    for (int t = 0; t < T; t++) {
        const int pos = start_pos + t;
        if (L->rope_q_cos)
            for (int hh = 0; hh < H; hh++) rope_hf_row(qr + ((size_t)t * H + hh) * dhr, L->rope_q_cos, L->rope_q_sin, dhr, pos);
        if (L->rope_k_cos)
            for (int hh = 0; hh < Hkv; hh++) rope_hf_row(kr + ((size_t)t * Hkv + hh) * dhr, L->rope_k_cos, L->rope_k_sin, dhr, pos);
        /* build_qkv (build_qkv_fp32.cu:8-24): K row per kv head [k | kr], V row per kv head */
        float* krow = m->kc[l] + (size_t)pos * Hkv * dq;
        for (int hh = 0; hh < Hkv; hh++) {
            memcpy(krow + hh * dq, k + ((size_t)t * Hkv + hh) * dh, (size_t)dh * 4);
            memcpy(krow + hh * dq + dh, kr + ((size_t)t * Hkv + hh) * dhr, (size_t)dhr * 4);
        }
        memcpy(m->vc[l] + (size_t)pos * Hkv * dh, v + (size_t)t * Hkv * dh, (size_t)Hkv * dh * 4);
        if (qkv) {
            memcpy(kcur + (size_t)t * Hkv * dq, krow, (size_t)Hkv * dq * 4);
            memcpy(vcur + (size_t)t * Hkv * dh, v + (size_t)t * Hkv * dh, (size_t)Hkv * dh * 4);
            for (int hh = 0; hh < Hkv; hh++) {
                const size_t r = (size_t)pos * Hkv + hh;
                orc_kv_quantize(ORC_KVF_Q2_1, k + ((size_t)t * Hkv + hh) * dh, m->kq[l] + r * (dh / 32) * 10, dh);
                orc_kv_quantize(ORC_KVF_Q1_0, v + ((size_t)t * Hkv + hh) * dh, m->vq[l] + r * (dh / 32) * 6, dh);
                /* from now on the row is read through the packed cache */
                orc_kv_dequant(ORC_KVF_Q2_1, m->kq[l] + r * (dh / 32) * 10, m->kc[l] + r * dq, dh);
                orc_kv_dequant(ORC_KVF_Q1_0, m->vq[l] + r * (dh / 32) * 6, m->vc[l] + r * dh, dh);
            }
        }
    }
    {   /* query rows are independent: rows t = w, w + nw, ... per worker */
        rmla_rows_job jobs[64];
        pthread_t th[64];
        int nw = nt > 0 ? nt : orc_num_threads();
        if (nw > T) nw = T;
        if (nw > 64) nw = 64;
        for (int w = 0; w < nw; w++) {
            jobs[w] = (rmla_rows_job){q, qr, m->kc[l], m->vc[l], kcur, vcur, att, H, Hkv, dh, dhr, T, start_pos, w, nw};
            if (w) pthread_create(&th[w], NULL, rmla_rows_worker, &jobs[w]);
        }
        rmla_rows_worker(&jobs[0]);
        for (int w = 1; w < nw; w++) pthread_join(th[w], NULL);
    }
    free(kcur);
    free(vcur);
    orc_linear(L->c_proj, L->qt, att, tmp, T, d, H * dh, nt);                   /* :87 (out of place) */
    orc_add(h, h, tmp, T * d);
    free(a); free(cq); free(q); free(k); free(v); free(qr); free(kr); free(att); free(tmp);
}

int orc_jamba_forward(orc_jamba* m, const int* ids, int T, int start_pos, float* logits, int last_only) {
    const orc_jamba_cfg* c = &m->c;
    const int d = c->dim, nt = c->nthreads, hd = c->hidden;
    if (start_pos < 0 || start_pos + T > c->max_seq) return -3;
    if (start_pos == 0)
        for (int l = 0; l < c->n_layers; l++)
            if (m->lcs[l]) {
                memset(m->lcs[l], 0, (size_t)c->n_heads * c->head_dim * 4);
                memset(m->wcs[l], 0, (size_t)c->n_heads * c->head_dim * 4);
            }
    float* h = (float*)malloc((size_t)T * d * 4);
    float* a = (float*)malloc((size_t)T * d * 4);
    float* g = (float*)malloc((size_t)T * hd * 4);
    float* u = (float*)malloc((size_t)T * hd * 4);
    orc_embedding(c->wte, c->qt_wte, ids, h, T, d);
    for (int l = 0; l < c->n_layers; l++) {
        const orc_jamba_layer_w* L = &c->layers[l];
        if (L->type == ORC_JAMBA_SSM) jamba_ssm(m, l, h, T);
        else jamba_rmla(m, l, h, T, start_pos);
        memcpy(a, h, (size_t)T * d * 4);                                        /* MLP */
        orc_layer_norm(a, L->ln2, T, d, 1e-5f);
        orc_linear(L->w1, L->qt, a, g, T, hd, d, nt);
        orc_linear(L->w3, L->qt, a, u, T, hd, d, nt);
        orc_silu_mul(g, g, u, T * hd);
        orc_linear(L->w2, L->qt, g, a, T, d, hd, nt);
        orc_add(h, h, a, T * d);
    }
    if (c->ln_f) orc_layer_norm(h, c->ln_f, T, d, 1e-5f);                       /* name is not "llama" */
    const void* lm = c->lm_head ? c->lm_head : c->wte;
    int qlm = c->lm_head ? c->qt_lm : c->qt_wte;
    if (last_only) orc_linear(lm, qlm, h + (size_t)(T - 1) * d, logits, 1, c->vocab, d, nt);
    else orc_linear(lm, qlm, h, logits, T, c->vocab, d, nt);
    free(h); free(a); free(g); free(u);
    return 0;
}

static int jamba_gen(orc_jamba* m, const int* prompt, int n_prompt, int steps, int* out_ids, int recompute) {
    int V = m->c.vocab;
    int* gen = (int*)malloc(sizeof(int) * (n_prompt + steps));
    memcpy(gen, prompt, sizeof(int) * n_prompt);
    float* logits = (float*)malloc((size_t)V * 4);
    int len = n_prompt, rc = 0;
    for (int step = 0; step < steps; step++) {
        if (recompute || step == 0) rc = orc_jamba_forward(m, gen, len, 0, logits, 1);
        else rc = orc_jamba_forward(m, gen + len - 1, 1, len - 1, logits, 1);
        if (rc) break;
        int nx = orc_argmax(logits, V);
        gen[len++] = nx;
        out_ids[step] = nx;
    }
    free(gen);
    free(logits);
    return rc;
}

int orc_jamba_generate(orc_jamba* m, const int* p, int n, int steps, int* out) { return jamba_gen(m, p, n, steps, out, 0); }
int orc_jamba_generate_recompute(orc_jamba* m, const int* p, int n, int steps, int* out) {
    return jamba_gen(m, p, n, steps, out, 1);
}
