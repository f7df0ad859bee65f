// Per-token glue of the decode step (RMSNorm, LayerNorm, RoPE, embedding,
// SiLU*up, add, saxpy, greedy argmax) and the library's runtime helpers.
#include "rina_common.hpp"
#include "kv_formats.hpp"
#include <mutex>
#include <vector>

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = 0.f;
    const int nw = (blockDim.x + 63) >> 6;
    for (int i = 0; i < nw; i++) t += red[i];
    return t;
}

// ops/rms_norm.cu:5-29
__global__ __launch_bounds__(256) void rms_norm_kernel(const float* x, float* out, const float* w, int d, float eps) {
    __shared__ float red[4];
    const float* row = x + (int64_t)blockIdx.x * d;
    float* orow = out + (int64_t)blockIdx.x * d;
    float ss = 0.f;
    for (int i = threadIdx.x; i < d; i += blockDim.x) ss = fmaf(row[i], row[i], ss);
    ss = block_sum(ss, red);
    float inv = 1.0f / sqrtf(ss / (float)d + eps);
    for (int i = threadIdx.x; i < d; i += blockDim.x) orow[i] = row[i] * inv * w[i];
}

// The same RMSNorm for rows of d <= 1024 NV values (d % 4 == 0, 16-byte
// aligned rows): each thread holds its NV float4 of the row in registers,
// so the row is read once with 16-byte loads (prompt rows before a matmul).
template <int NV>
__global__ __launch_bounds__(256) void rms_norm_vec_kernel(const float* x, float* out, const float* w, int d, float eps) {
    __shared__ float red[4];
    const f32x4* row = (const f32x4*)(x + (int64_t)blockIdx.x * d);
    f32x4* orow = (f32x4*)(out + (int64_t)blockIdx.x * d);
    const int n4 = d >> 2;
    f32x4 v[NV];
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const int i = threadIdx.x + 256 * k;
        v[k] = i < n4 ? gld(row + i) : f32x4{0.f, 0.f, 0.f, 0.f};
        ss = fmaf(v[k].x, v[k].x, ss);
        ss = fmaf(v[k].y, v[k].y, ss);
        ss = fmaf(v[k].z, v[k].z, ss);
        ss = fmaf(v[k].w, v[k].w, ss);
    }
    ss = block_sum(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)d + eps);
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const int i = threadIdx.x + 256 * k;
        if (i < n4) {
            const f32x4 g = gld((const f32x4*)w + i);
            gst(orow + i, f32x4{v[k].x * inv * g.x, v[k].y * inv * g.y, v[k].z * inv * g.z, v[k].w * inv * g.w});
        }
    }
}

// kernels/pytorch_ln_kernel.cu:4-35 (biased variance; two-pass form)
__global__ __launch_bounds__(256) void layer_norm_kernel(const float* x, float* out, const float* w, int d, float eps) {
    __shared__ float red[4];
    const float* row = x + (int64_t)blockIdx.x * d;
    float* orow = out + (int64_t)blockIdx.x * d;
    float s = 0.f;
    for (int i = threadIdx.x; i < d; i += blockDim.x) s += row[i];
    float mean = block_sum(s, red) / (float)d;
    float v = 0.f;
    for (int i = threadIdx.x; i < d; i += blockDim.x) {
        float t = row[i] - mean;
        v = fmaf(t, t, v);
    }
    float var = block_sum(v, red) / (float)d;
    float inv = 1.0f / sqrtf(var + eps);
    for (int i = threadIdx.x; i < d; i += blockDim.x) orow[i] = (row[i] - mean) * inv * (w ? w[i] : 1.0f);
}

// ops/rope.cu:125-149 (pairs i, i+d/2) and :212-234 (pairs 2i, 2i+1)
__global__ void rope_kernel(float* x, const float* ct, const float* st, int T, int H, int d, int start_pos,
                            const int* d_pos, int hf) {
    const int half = d / 2;
    int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= (int64_t)T * H * half) return;
    int i = (int)(p % half);
    int64_t th = p / half;
    int t = (int)(th / H);
    int pos = read_pos(start_pos, d_pos) + t;
    float c = ct[(int64_t)pos * half + i], s = st[(int64_t)pos * half + i];
    float* row = x + th * d;
    int i0 = hf ? 2 * i : i, i1 = hf ? 2 * i + 1 : i + half;
    float x0 = row[i0], x1 = row[i1];
    row[i0] = x0 * c - x1 * s;
    row[i1] = x0 * s + x1 * c;
}

// ops/embedding.cu:6-230: row lookup with per-format dequant; Q2_K rows are
// row-aligned (ceil(d/256) blocks per row, ops/embedding.cu:80-81).  With
// vocab > 0 an id outside [0, vocab) is clamped into it, so a bad id read
// from device memory never indexes past the table (the reference reads it
// unchecked; host prompts are rejected before launch by the engine).
__global__ void embedding_kernel(const uint8_t* w, int qt, const int* ids, const int* d_pos, float* out, int d,
                                 int vocab) {
    const int t = blockIdx.x;
    const int off = d_pos ? *d_pos : 0;
    int id = ids[off + t];
    if (id < 0) id = 0;
    if (vocab > 0 && id >= vocab) id = vocab - 1;
    float* o = out + (int64_t)t * d;
    const uint8_t* row;
    if (qt == RINA_QT_Q4_0) row = w + (int64_t)id * (d / 32) * 18;
    else if (qt == RINA_QT_Q4_0F) row = w + (int64_t)id * (d / 32) * 20;
    else if (qt == RINA_QT_GGML_Q2_K) row = w + (int64_t)id * ((d + 255) / 256) * 84;
    else row = w + (int64_t)id * d * 4;
    for (int i = threadIdx.x; i < d; i += blockDim.x) o[i] = kvq::weight_elem(qt, row, i);
}

__global__ void silu_mul_kernel(float* o, const float* g, const float* u, int64_t n) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) o[i] = (g[i] / (1.0f + expf(-g[i]))) * u[i];
}
__global__ void add_kernel(float* c, const float* a, const float* b, int64_t n) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) c[i] = a[i] + b[i];
}
__global__ void saxpy_kernel(float* d, const float* s, float p, int64_t n) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) d[i] += p * s[i];
}

// Greedy argmax (main.cpp:139-146): strict ">" from -1e10, lowest index on
// ties.  Candidates are packed into one 64-bit key (argmax_key) and merged
// with a 64-bit atomicMax into a key slot that the finishing kernel reads
// and clears again.
__device__ unsigned long long g_argmax_key = 0ull;   // slot of rina_hip_argmax (one per device)

__device__ __forceinline__ unsigned long long cand(float v, int i) { return argmax_cand(v, i); }

// A few workgroups (one 64-bit atomic each, after a wave + LDS reduction)
// cover x with 16-byte loads; many same-address atomics serialize.
__global__ __launch_bounds__(256) void argmax_partial_kernel(const float* x, int n, unsigned long long* key) {
    __shared__ unsigned long long red[4];
    unsigned long long best = 0ull;
    const int tid = threadIdx.x;
    const int stride = gridDim.x * blockDim.x;
    const int n4 = ((uintptr_t)x % 16 == 0) ? n / 4 : 0;
    const f32x4* x4 = (const f32x4*)x;
    for (int i = blockIdx.x * blockDim.x + tid; i < n4; i += stride) {
        const f32x4 v = gld(x4 + i);
        best = umax64(best, umax64(umax64(cand(v.x, 4 * i), cand(v.y, 4 * i + 1)),
                                   umax64(cand(v.z, 4 * i + 2), cand(v.w, 4 * i + 3))));
    }
    for (int i = 4 * n4 + blockIdx.x * blockDim.x + tid; i < n; i += stride) best = umax64(best, cand(gld(x + i), i));
    for (int off = 32; off > 0; off >>= 1) best = umax64(best, __shfl_xor(best, off));
    if ((tid & 63) == 0) red[tid >> 6] = best;
    __syncthreads();
    if (tid == 0) {
        best = umax64(umax64(red[0], red[1]), umax64(red[2], red[3]));
        if (best) atomicMax(key, best);
    }
}

__global__ void argmax_finish_kernel(int* out_idx, int* ids_out, int* d_pos, unsigned long long* key) {
    unsigned long long k = *key;
    *key = 0ull;
    int idx = argmax_index(k);
    if (out_idx) *out_idx = idx;
    if (d_pos) {
        int p = *d_pos;
        if (ids_out) ids_out[p + 1] = idx;
        *d_pos = p + 1;
    }
}

// The greedy step's tail in one launch: the winner of nkeys argmax keys
// (the per-workgroup keys of a fused LM head, or a key slot, cleared again
// when `reset`), then what argmax_finish_kernel does with it (out_idx, the
// id after the device position, the position advanced), then the
// embedding row of that id into h: the next decode step's input
// (ops/embedding.cu:6-230 via kvq::weight_elem, ids outside the vocabulary
// clamped as embedding_kernel does).
__global__ __launch_bounds__(256) void argmax_embed_kernel(unsigned long long* keys, int nkeys, int reset, int* out_idx,
                                                           int* ids_out, int* d_pos, const uint8_t* w, int qt,
                                                           float* h, int d, int vocab) {
    __shared__ unsigned long long red[4];
    __shared__ int s_id;
    const int tid = threadIdx.x;
    unsigned long long best = 0ull;
    for (int i = tid; i < nkeys; i += 256) best = umax64(best, gld(keys + i));
    for (int off = 32; off > 0; off >>= 1) best = umax64(best, __shfl_xor(best, off));
    if ((tid & 63) == 0) red[tid >> 6] = best;
    __syncthreads();
    if (tid == 0) {
        const int idx = argmax_index(umax64(umax64(red[0], red[1]), umax64(red[2], red[3])));
        if (out_idx) *out_idx = idx;
        if (d_pos) {
            const int p = *d_pos;
            if (ids_out) ids_out[p + 1] = idx;
            *d_pos = p + 1;
        }
        s_id = idx;
    }
    __syncthreads();
    if (reset)
        for (int i = tid; i < nkeys; i += 256) keys[i] = 0ull;
    int id = s_id;
    if (id < 0) id = 0;
    if (vocab > 0 && id >= vocab) id = vocab - 1;
    const uint8_t* row;
    if (qt == RINA_QT_Q4_0) row = w + (int64_t)id * (d / 32) * 18;
    else if (qt == RINA_QT_Q4_0F) row = w + (int64_t)id * (d / 32) * 20;
    else if (qt == RINA_QT_GGML_Q2_K) row = w + (int64_t)id * ((d + 255) / 256) * 84;
    else row = w + (int64_t)id * d * 4;
    for (int i = tid; i < d; i += 256) h[i] = kvq::weight_elem(qt, row, i);
}

// Streaming-read probe: every lane sums 16-byte non-temporal loads of its
// grid-stride slice, four in flight; one float per workgroup is written so
// the loads cannot be dropped.  Measures what a plain read of `bytes`
// costs in one launch (the ceiling a matvec of the same size could reach).
__global__ __launch_bounds__(256) void read_probe_kernel(const f32x4* src, int64_t n4, float* sink) {
    __shared__ float red[4];
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    float acc = 0.f;
    for (; i + 3 * stride < n4; i += 4 * stride) {
        const f32x4 a = gld_nt(src + i), b = gld_nt(src + i + stride), c = gld_nt(src + i + 2 * stride),
                    d = gld_nt(src + i + 3 * stride);
        acc += (a.x + b.y) + (c.z + d.w);
    }
    for (; i < n4; i += stride) acc += gld_nt(src + i).x;
    acc = wave_sum(acc);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) sink[blockIdx.x] = (red[0] + red[1]) + (red[2] + red[3]);
}

unsigned blocks_for(int64_t n, int bs) { return (unsigned)((n + bs - 1) / bs); }

struct DevState {
    int cus = 0;
};
DevState g_dev[64];
std::mutex g_mu;

// Library scratch, one buffer per (device, stream): work on different
// streams never shares it, and work on one stream is ordered.  A buffer
// that must grow is replaced by one of at least twice its size; the old
// one may still be read by queued work, so it is kept (retired) until the
// process ends: at most log2 of the largest request buffers per stream.
struct ScratchSlot {
    int dev;
    hipStream_t st;
    void* p;
    size_t bytes;
};
std::vector<ScratchSlot> g_scratch;
std::vector<void*> g_retired;

}  // namespace

int rina_num_cus() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!g_dev[dev].cus) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        g_dev[dev].cus = n;
    }
    return g_dev[dev].cus;
}

void* rina_scratch(size_t bytes, hipStream_t st) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return nullptr;
    std::lock_guard<std::mutex> lk(g_mu);
    for (ScratchSlot& s : g_scratch) {
        if (s.dev != dev || s.st != st) continue;
        if (s.bytes >= bytes) return s.p;
        size_t nb = bytes > 2 * s.bytes ? bytes : 2 * s.bytes;
        void* p = nullptr;
        if (hipMalloc(&p, nb) != hipSuccess) return nullptr;
        g_retired.push_back(s.p);
        s.p = p;
        s.bytes = nb;
        return p;
    }
    void* p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess) return nullptr;
    g_scratch.push_back({dev, st, p, bytes});
    return p;
}

extern "C" int rina_hip_rms_norm(const float* x, float* out, const float* w, int n, int d, float eps, void* stream) {
    if (!x || !out || !w || n < 1 || d < 1) return RINA_ERR_ARG;
    const bool vec = d % 4 == 0 && d <= 8192 && (((uintptr_t)x | (uintptr_t)out | (uintptr_t)w) % 16) == 0;
    const int nv = (d / 4 + 255) / 256;
    hipStream_t st = as_stream(stream);
    if (vec && nv <= 1) hipLaunchKernelGGL(rms_norm_vec_kernel<1>, dim3(n), dim3(256), 0, st, x, out, w, d, eps);
    else if (vec && nv <= 2) hipLaunchKernelGGL(rms_norm_vec_kernel<2>, dim3(n), dim3(256), 0, st, x, out, w, d, eps);
    else if (vec && nv <= 4) hipLaunchKernelGGL(rms_norm_vec_kernel<4>, dim3(n), dim3(256), 0, st, x, out, w, d, eps);
    else if (vec) hipLaunchKernelGGL(rms_norm_vec_kernel<8>, dim3(n), dim3(256), 0, st, x, out, w, d, eps);
    else hipLaunchKernelGGL(rms_norm_kernel, dim3(n), dim3(256), 0, st, x, out, w, d, eps);
    RINA_LAUNCH_CHECK();
    return RINA_OK;
}

extern "C" int rina_hip_layer_norm(const float* x, float* out, const float* w, int n, int d, float eps, void* stream) {
    if (!x || !out || n < 1 || d < 1) return RINA_ERR_ARG;
    hipLaunchKernelGGL(layer_norm_kernel, dim3(n), dim3(256), 0, as_stream(stream), x, out, w, d, eps);
    RINA_LAUNCH_CHECK();
    return RINA_OK;
}

extern "C" int rina_hip_rope(float* x, const float* ct, const float* st, int T, int H, int d, int start_pos,
                             const int* d_pos, int hf, void* stream) {
    if (!x || !ct || !st || T < 1 || H < 1 || d < 2 || (d & 1)) return RINA_ERR_ARG;
    int64_t n = (int64_t)T * H * (d / 2);
    hipLaunchKernelGGL(rope_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, as_stream(stream), x, ct, st, T, H, d,
                       start_pos, d_pos, hf);
    RINA_LAUNCH_CHECK();
    return RINA_OK;
}

extern "C" int rina_hip_embedding(const void* w, int qt, const int* ids, const int* d_pos, float* out, int n, int d,
                                  int vocab, void* stream) {
    if (!w || !ids || !out || n < 1 || d < 1) return RINA_ERR_ARG;
    if (qt != RINA_QT_FP32 && qt != RINA_QT_Q4_0 && qt != RINA_QT_Q4_0F && qt != RINA_QT_GGML_Q2_K)
        return RINA_ERR_QTYPE;
    if ((qt == RINA_QT_Q4_0 || qt == RINA_QT_Q4_0F) && d % 32) return RINA_ERR_SHAPE;
    hipLaunchKernelGGL(embedding_kernel, dim3(n), dim3(256), 0, as_stream(stream), (const uint8_t*)w, qt, ids, d_pos,
                       out, d, vocab);
    RINA_LAUNCH_CHECK();
    return RINA_OK;
}

extern "C" int rina_hip_silu_mul(float* o, const float* g, const float* u, int64_t n, void* stream) {
    if (!o || !g || !u || n < 0) return RINA_ERR_ARG;
    if (!n) return RINA_OK;
    hipLaunchKernelGGL(silu_mul_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, as_stream(stream), o, g, u, n);
    RINA_LAUNCH_CHECK();
    return RINA_OK;
}

extern "C" int rina_hip_add(float* c, const float* a, const float* b, int64_t n, void* stream) {
    if (!c || !a || !b || n < 0) return RINA_ERR_ARG;
    if (!n) return RINA_OK;
    hipLaunchKernelGGL(add_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, as_stream(stream), c, a, b, n);
    RINA_LAUNCH_CHECK();
    return RINA_OK;
}

extern "C" int rina_hip_saxpy(float* d, const float* s, float p, int64_t n, void* stream) {
    if (!d || !s || n < 0) return RINA_ERR_ARG;
    if (!n) return RINA_OK;
    hipLaunchKernelGGL(saxpy_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, as_stream(stream), d, s, p, n);
    RINA_LAUNCH_CHECK();
    return RINA_OK;
}

namespace {
int argmax_launch(const float* x, int n, int* out_idx, int* ids_out, int* d_pos, unsigned long long* key,
                  hipStream_t st) {
    int grid = (n + 1023) / 1024;
    if (grid > 64) grid = 64;
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(grid), dim3(256), 0, st, x, n, key);
    RINA_LAUNCH_CHECK();
    hipLaunchKernelGGL(argmax_finish_kernel, dim3(1), dim3(1), 0, st, out_idx, ids_out, d_pos, key);
    RINA_LAUNCH_CHECK();
    return RINA_OK;
}

// device address of g_argmax_key, looked up once per device with that
// device current (host code must never pass the symbol itself)
unsigned long long* g_key_addr[64];
std::mutex g_key_mu;
}  // namespace

extern "C" int rina_hip_argmax(const float* x, int n, int* out_idx, int* ids_out, int* d_pos, void* stream) {
    if (!x || n < 1 || (!out_idx && !d_pos)) return RINA_ERR_ARG;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return RINA_ERR_HIP;
    unsigned long long* key;
    {
        std::lock_guard<std::mutex> lk(g_key_mu);
        if (!g_key_addr[dev]) {
            void* p = nullptr;
            if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_argmax_key)) != hipSuccess || !p) return RINA_ERR_HIP;
            g_key_addr[dev] = (unsigned long long*)p;
        }
        key = g_key_addr[dev];
    }
    return argmax_launch(x, n, out_idx, ids_out, d_pos, key, as_stream(stream));
}

extern "C" int rina_hip_argmax_partial(const float* x, int n, void* key_slot, void* stream) {
    if (!x || n < 1 || !key_slot || (uintptr_t)key_slot % 8) return RINA_ERR_ARG;
    int grid = (n + 1023) / 1024;
    if (grid > 64) grid = 64;
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(grid), dim3(256), 0, as_stream(stream), x, n,
                       (unsigned long long*)key_slot);
    RINA_LAUNCH_CHECK();
    return RINA_OK;
}

extern "C" int rina_hip_argmax_embed(void* keys, int nkeys, int reset, int* out_idx, int* ids_out, int* d_pos,
                                     const void* emb, int emb_qt, float* h, int d, int vocab, void* stream) {
    if (!keys || nkeys < 1 || (uintptr_t)keys % 8 || !emb || !h || d < 1 || vocab < 1) return RINA_ERR_ARG;
    if (emb_qt != RINA_QT_FP32 && emb_qt != RINA_QT_Q4_0 && emb_qt != RINA_QT_Q4_0F && emb_qt != RINA_QT_GGML_Q2_K)
        return RINA_ERR_QTYPE;
    if ((emb_qt == RINA_QT_Q4_0 || emb_qt == RINA_QT_Q4_0F) && d % 32) return RINA_ERR_SHAPE;
    hipLaunchKernelGGL(argmax_embed_kernel, dim3(1), dim3(256), 0, as_stream(stream), (unsigned long long*)keys,
                       nkeys, reset, out_idx, ids_out, d_pos, (const uint8_t*)emb, emb_qt, h, d, vocab);
    RINA_LAUNCH_CHECK();
    return RINA_OK;
}

extern "C" int rina_hip_argmax_ws(const float* x, int n, int* out_idx, int* ids_out, int* d_pos, void* key_slot,
                                  void* stream) {
    if (!x || n < 1 || (!out_idx && !d_pos) || !key_slot || (uintptr_t)key_slot % 8) return RINA_ERR_ARG;
    return argmax_launch(x, n, out_idx, ids_out, d_pos, (unsigned long long*)key_slot, as_stream(stream));
}

extern "C" int rina_hip_read_probe(const void* src, int64_t bytes, int grid, float* sink, void* stream) {
    if (!src || !sink || bytes < 16 || grid < 1 || (uintptr_t)src % 16) return RINA_ERR_ARG;
    hipLaunchKernelGGL(read_probe_kernel, dim3(grid), dim3(256), 0, as_stream(stream), (const f32x4*)src, bytes / 16,
                       sink);
    RINA_LAUNCH_CHECK();
    return RINA_OK;
}

extern "C" const char* rina_hip_version(void) { return "rina-mi355x hip 0.1 (gfx950)"; }
