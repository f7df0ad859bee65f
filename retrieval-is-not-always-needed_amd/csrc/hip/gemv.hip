// Quantized matvec for gfx950: RINA Q4_0 / Q4_0F, GGML Q2_K (flat element
// indexing) and fp32, M = 1 decode path plus a tiled M > 1 path.
//
// Decode (M = 1) design, HBM-bound:
//   * A workgroup owns a tile of R consecutive weight rows.  Rows are
//     contiguous in memory, so the tile is one contiguous byte range; the
//     256 threads copy it to LDS with coalesced 16-byte loads (the 18/20/84
//     byte blocks never have to be 16-byte aligned in HBM).  The next tile's
//     loads are issued before the current tile is computed (register
//     double-buffering, one LDS barrier per tile).
//   * Lane l of a wave owns the same block columns of every row, so its 32
//     activation values live in registers for the whole launch, together
//     with their sum: sum_i x_i (q_i - 7) s = s (sum_i q_i x_i - 7 sum_i x_i).
//   * Nibbles are split with two masks and converted with v_cvt_f32_ubyteN.
//   * Row sums reduce through DPP (no LDS); for K > 64 blocks, 2 or 4 waves
//     split a row and combine through a small LDS array.
// Epilogues fuse the reference's follow-up launches (residual add, SiLU*up).
#include "rina_common.hpp"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWG = 256;
constexpr int kMaxChunks = 4;              // 16-byte chunks per thread per tile
constexpr int kTileBytes = kWG * kMaxChunks * 16;   // 16 KiB per tile (all matrices)

enum { FMT_Q4_0 = 0, FMT_Q4_0F = 1, FMT_Q2_K = 2 };

struct GemvSeg {
    const uint8_t* w;
    const uint8_t* w2;
    float* y;
    int N;
    int tile0;
};

struct GemvArgs {
    GemvSeg seg[3];
    int nseg;
    const float* x;
    int K;
    int R;            // rows per tile
    int total_tiles;
    int epi;
    int rowbytes;     // Q4 formats: bytes per row
    int slot;         // LDS bytes per matrix slot (16-byte multiple)
};

__device__ __forceinline__ void tile_of(const GemvArgs& a, int t, int& s, int& n0, int& rows) {
    s = 0;
    if (a.nseg > 1 && t >= a.seg[1].tile0) s = 1;
    if (a.nseg > 2 && t >= a.seg[2].tile0) s = 2;
    n0 = (t - a.seg[s].tile0) * a.R;
    rows = min(a.R, a.seg[s].N - n0);
}

// byte range [start, start+len) of the tile's rows inside the weight stream
template <int FMT>
__device__ __forceinline__ void tile_bytes(const GemvArgs& a, int n0, int rows, int64_t& start, int64_t& len) {
    if (FMT == FMT_Q2_K) {
        int64_t e0 = (int64_t)n0 * a.K, e1 = (int64_t)(n0 + rows) * a.K;
        int64_t b0 = e0 >> 8, b1 = (e1 + 255) >> 8;
        start = b0 * 84;
        len = (b1 - b0) * 84;
    } else {
        start = (int64_t)n0 * a.rowbytes;
        len = (int64_t)rows * a.rowbytes;
    }
}

template <int FMT, int NMAT>
__device__ __forceinline__ void tile_load(const GemvArgs& a, int t, u32x4 (&pre)[kMaxChunks]) {
    int s, n0, rows;
    tile_of(a, t, s, n0, rows);
    int64_t start, len;
    tile_bytes<FMT>(a, n0, rows, start, len);
    const int tid = threadIdx.x;
    int nch[2];
    const uint8_t* base[2];
#pragma unroll
    for (int m = 0; m < NMAT; m++) {
        const uint8_t* g = (m == 0 ? a.seg[s].w : a.seg[s].w2) + start;
        int lead = (int)((uintptr_t)g & 15);
        base[m] = g - lead;
        nch[m] = (int)((lead + len + 15) >> 4);
    }
#pragma unroll
    for (int i = 0; i < kMaxChunks; i++) {
        int c = tid + i * kWG;
        int m = 0;
        if (NMAT == 2 && c >= nch[0]) { c -= nch[0]; m = 1; }
        if (c < nch[m]) pre[i] = __builtin_nontemporal_load((const u32x4*)(base[m]) + c);
    }
}

template <int FMT, int NMAT>
__device__ __forceinline__ void tile_store(const GemvArgs& a, int t, const u32x4 (&pre)[kMaxChunks], uint8_t* buf) {
    int s, n0, rows;
    tile_of(a, t, s, n0, rows);
    int64_t start, len;
    tile_bytes<FMT>(a, n0, rows, start, len);
    const int tid = threadIdx.x;
    int nch[2];
#pragma unroll
    for (int m = 0; m < NMAT; m++) {
        const uint8_t* g = (m == 0 ? a.seg[s].w : a.seg[s].w2) + start;
        int lead = (int)((uintptr_t)g & 15);
        nch[m] = (int)((lead + len + 15) >> 4);
    }
#pragma unroll
    for (int i = 0; i < kMaxChunks; i++) {
        int c = tid + i * kWG;
        int m = 0;
        if (NMAT == 2 && c >= nch[0]) { c -= nch[0]; m = 1; }
        if (c < nch[m]) *(u32x4*)(buf + m * a.slot + c * 16) = pre[i];
    }
}

__device__ __forceinline__ uint32_t lds_u32(const uint8_t* p) { return *(const uint32_t*)p; }
__device__ __forceinline__ uint32_t lds_u16(const uint8_t* p) { return *(const uint16_t*)p; }

__device__ __forceinline__ uint32_t funnel(uint32_t lo, uint32_t hi, uint32_t sh) {
    return (uint32_t)((((uint64_t)hi << 32) | lo) >> sh);
}

// sum_i q_i x_i over one 32-value block whose 16 nibble bytes are nib[0..3]
__device__ __forceinline__ float q4_dot(const uint32_t (&nib)[4], const float* x) {
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int d = 0; d < 4; d++) {
        uint32_t lo = nib[d] & 0x0F0F0F0Fu, hi = (nib[d] >> 4) & 0x0F0F0F0Fu;
        a0 = fmaf((float)(lo & 0xFF), x[8 * d + 0], a0);
        a1 = fmaf((float)(hi & 0xFF), x[8 * d + 1], a1);
        a0 = fmaf((float)((lo >> 8) & 0xFF), x[8 * d + 2], a0);
        a1 = fmaf((float)((hi >> 8) & 0xFF), x[8 * d + 3], a1);
        a0 = fmaf((float)((lo >> 16) & 0xFF), x[8 * d + 4], a0);
        a1 = fmaf((float)((hi >> 16) & 0xFF), x[8 * d + 5], a1);
        a0 = fmaf((float)(lo >> 24), x[8 * d + 6], a0);
        a1 = fmaf((float)(hi >> 24), x[8 * d + 7], a1);
    }
    return a0 + a1;
}

// sum_i q_i x_i over a 16-value Q2_K unit: qs bytes q[0..3], shift 2g
__device__ __forceinline__ float q2_dot(const uint32_t (&q)[4], uint32_t sh, const float* x) {
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int d = 0; d < 4; d++) {
        uint32_t t = (q[d] >> sh) & 0x03030303u;
        a0 = fmaf((float)(t & 0xFF), x[4 * d + 0], a0);
        a1 = fmaf((float)((t >> 8) & 0xFF), x[4 * d + 1], a1);
        a0 = fmaf((float)((t >> 16) & 0xFF), x[4 * d + 2], a0);
        a1 = fmaf((float)(t >> 24), x[4 * d + 3], a1);
    }
    return a0 + a1;
}

__device__ __forceinline__ float silu_mul(float g, float u) { return (g / (1.0f + expf(-g))) * u; }

template <int NMAT>
__device__ __forceinline__ void epilogue(const GemvArgs& a, int s, int n, const float (&v)[2]) {
    float* y = a.seg[s].y + n;
    if (NMAT == 2) *y = silu_mul(v[0], v[1]);
    else if (a.epi == RINA_EPI_ADD) *y = *y + v[0];
    else *y = v[0];
}

// UNIT: values per lane work unit (32 for Q4 blocks, 16 for Q2_K units)
template <int FMT, int WPR, int CPL, int NMAT>
__global__ __launch_bounds__(kWG) void gemv_quant_kernel(GemvArgs a) {
    constexpr int UNIT = (FMT == FMT_Q2_K) ? 16 : 32;
    constexpr int RPI = 4 / WPR;
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int rs = wave / WPR, cp = wave % WPR;
    const int K = a.K;
    const int nunits = K / UNIT;

    // activation columns owned by this lane
    float xr[CPL][UNIT];
    float xs[CPL];
#pragma unroll
    for (int j = 0; j < CPL; j++) {
        int u = (cp * CPL + j) * 64 + lane;
        xs[j] = 0.f;
        if (u < nunits) {
            const f32x4* xp = (const f32x4*)(a.x + (int64_t)u * UNIT);
#pragma unroll
            for (int i = 0; i < UNIT / 4; i++) {
                f32x4 v = xp[i];
                xr[j][4 * i + 0] = v.x; xr[j][4 * i + 1] = v.y;
                xr[j][4 * i + 2] = v.z; xr[j][4 * i + 3] = v.w;
            }
#pragma unroll
            for (int i = 0; i < UNIT; i++) xs[j] += xr[j][i];
        } else {
#pragma unroll
            for (int i = 0; i < UNIT; i++) xr[j][i] = 0.f;
        }
    }

    const int bufbytes = NMAT * a.slot;
    float* red = (float*)(smem + 2 * bufbytes);   // [NMAT][R][WPR]

    u32x4 pre[kMaxChunks];
    int t = blockIdx.x;
    if (t < a.total_tiles) tile_load<FMT, NMAT>(a, t, pre);
    int b = 0;
    for (; t < a.total_tiles; t += gridDim.x, b ^= 1) {
        uint8_t* buf = smem + b * bufbytes;
        tile_store<FMT, NMAT>(a, t, pre, buf);
        __syncthreads();
        int tn = t + gridDim.x;
        if (tn < a.total_tiles) tile_load<FMT, NMAT>(a, tn, pre);

        int s, n0, rows;
        tile_of(a, t, s, n0, rows);
        int64_t start, len;
        tile_bytes<FMT>(a, n0, rows, start, len);
        int lead[2];
#pragma unroll
        for (int m = 0; m < NMAT; m++)
            lead[m] = (int)((uintptr_t)((m == 0 ? a.seg[s].w : a.seg[s].w2) + start) & 15);

        for (int r = rs; r < rows; r += RPI) {
            float v[2] = {0.f, 0.f};
#pragma unroll
            for (int m = 0; m < NMAT; m++) {
                const uint8_t* sl = buf + m * a.slot + lead[m];
                float part = 0.f;
#pragma unroll
                for (int j = 0; j < CPL; j++) {
                    int u = (cp * CPL + j) * 64 + lane;
                    if (u >= nunits) continue;
                    if (FMT == FMT_Q4_0F) {
                        const uint8_t* bp = sl + r * a.rowbytes + u * 20;
                        float sc = __uint_as_float(lds_u32(bp));
                        uint32_t nib[4];
#pragma unroll
                        for (int d = 0; d < 4; d++) nib[d] = lds_u32(bp + 4 + 4 * d);
                        float qx = q4_dot(nib, xr[j]);
                        part = fmaf(sc, fmaf(-7.0f, xs[j], qx), part);
                    } else if (FMT == FMT_Q4_0) {
                        int off = (int)((uintptr_t)(sl + r * a.rowbytes + u * 18) - (uintptr_t)smem);
                        float sc = f16_to_f32(lds_u16(smem + off));
                        int an = (off + 2) & ~3;
                        uint32_t sh = (uint32_t)((off + 2) & 3) * 8;
                        uint32_t dw[5];
#pragma unroll
                        for (int d = 0; d < 5; d++) dw[d] = lds_u32(smem + an + 4 * d);
                        uint32_t nib[4];
#pragma unroll
                        for (int d = 0; d < 4; d++) nib[d] = funnel(dw[d], dw[d + 1], sh);
                        float qx = q4_dot(nib, xr[j]);
                        part = fmaf(sc, fmaf(-7.0f, xs[j], qx), part);
                    } else {
                        // Q2_K unit u of row n0+r: flat element e = (n0+r)K + 16u
                        int64_t e = (int64_t)(n0 + r) * K + (int64_t)u * 16;
                        int lb = (int)((e >> 8) - (((int64_t)n0 * K) >> 8));
                        int inb = (int)(e & 255);
                        int page = inb >> 7, g = (inb >> 5) & 3, h2 = (inb >> 4) & 1;
                        const uint8_t* bp = sl + lb * 84;
                        uint32_t dd = lds_u32(bp + 80);
                        float dall = f16_to_f32(dd & 0xFFFF), dmin = f16_to_f32(dd >> 16);
                        uint32_t scb = bp[8 * page + 2 * g + h2];
                        uint32_t q[4];
#pragma unroll
                        for (int d = 0; d < 4; d++) q[d] = lds_u32(bp + 16 + 32 * page + 16 * h2 + 4 * d);
                        float qx = q2_dot(q, 2u * g, xr[j]);
                        float dl = dall * (float)(scb & 0xF), ml = dmin * (float)(scb >> 4);
                        part = fmaf(dl, qx, fmaf(-ml, xs[j], part));
                    }
                }
                v[m] = wave_sum(part);
            }
            if (WPR == 1) {
                if (lane == 0) epilogue<NMAT>(a, s, n0 + r, v);
            } else if (lane == 0) {
#pragma unroll
                for (int m = 0; m < NMAT; m++) red[(m * a.R + r) * WPR + cp] = v[m];
            }
        }
        if (WPR > 1) {
            __syncthreads();
            if (tid < rows) {
                float v[2] = {0.f, 0.f};
#pragma unroll
                for (int m = 0; m < NMAT; m++) {
                    float acc = 0.f;
#pragma unroll
                    for (int c = 0; c < WPR; c++) acc += red[(m * a.R + tid) * WPR + c];
                    v[m] = acc;
                }
                epilogue<NMAT>(a, s, n0 + tid, v);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// fp32 weights: a wave streams two rows at a time with 16-byte loads; the
// activation vector is staged once per workgroup in LDS.
// ---------------------------------------------------------------------------
struct F32Args {
    GemvSeg seg[3];
    int nseg;
    const float* x;
    int K;
    int total_rows;
    int epi;
};

// dot of one fp32 row with the LDS copy of x; 4 independent 16-byte loads
// per lane per step keep ~4 KiB per wave in flight.
template <bool VEC>
__device__ __forceinline__ float f32_row_dot(const float* w, const float* xl, int K, int lane) {
    float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
    if (VEC) {
        const f32x4* w4 = (const f32x4*)w;
        const f32x4* x4 = (const f32x4*)xl;
        const int n4 = K >> 2;
        int k = lane;
        for (; k + 192 < n4; k += 256) {
            f32x4 a0 = __builtin_nontemporal_load(w4 + k);
            f32x4 a1 = __builtin_nontemporal_load(w4 + k + 64);
            f32x4 a2 = __builtin_nontemporal_load(w4 + k + 128);
            f32x4 a3 = __builtin_nontemporal_load(w4 + k + 192);
            f32x4 b0 = x4[k], b1 = x4[k + 64], b2 = x4[k + 128], b3 = x4[k + 192];
            s0 = fmaf(b0.x, a0.x, s0); s0 = fmaf(b0.y, a0.y, s0); s0 = fmaf(b0.z, a0.z, s0); s0 = fmaf(b0.w, a0.w, s0);
            s1 = fmaf(b1.x, a1.x, s1); s1 = fmaf(b1.y, a1.y, s1); s1 = fmaf(b1.z, a1.z, s1); s1 = fmaf(b1.w, a1.w, s1);
            s2 = fmaf(b2.x, a2.x, s2); s2 = fmaf(b2.y, a2.y, s2); s2 = fmaf(b2.z, a2.z, s2); s2 = fmaf(b2.w, a2.w, s2);
            s3 = fmaf(b3.x, a3.x, s3); s3 = fmaf(b3.y, a3.y, s3); s3 = fmaf(b3.z, a3.z, s3); s3 = fmaf(b3.w, a3.w, s3);
        }
        for (; k < n4; k += 64) {
            f32x4 a0 = __builtin_nontemporal_load(w4 + k);
            f32x4 b0 = x4[k];
            s0 = fmaf(b0.x, a0.x, s0); s0 = fmaf(b0.y, a0.y, s0); s0 = fmaf(b0.z, a0.z, s0); s0 = fmaf(b0.w, a0.w, s0);
        }
    } else {
        for (int k = lane; k < K; k += 64) s0 = fmaf(xl[k], w[k], s0);
    }
    return (s0 + s1) + (s2 + s3);
}

template <int NMAT, bool VEC>
__global__ __launch_bounds__(kWG) void gemv_f32_kernel(F32Args a) {
    extern __shared__ __align__(16) float xs_lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int K = a.K;
    for (int i = tid; i < K; i += kWG) xs_lds[i] = a.x[i];
    __syncthreads();
    const int gw = blockIdx.x * 4 + wave, nw = gridDim.x * 4;
    for (int vr = gw; vr < a.total_rows; vr += nw) {
        int s = 0;
        if (a.nseg > 1 && vr >= a.seg[1].tile0) s = 1;
        if (a.nseg > 2 && vr >= a.seg[2].tile0) s = 2;
        int row = vr - a.seg[s].tile0;
        float v[2];
#pragma unroll
        for (int m = 0; m < NMAT; m++) {
            const float* w = (const float*)(m == 0 ? a.seg[s].w : a.seg[s].w2) + (int64_t)row * K;
            v[m] = wave_sum(f32_row_dot<VEC>(w, xs_lds, K, lane));
        }
        if (lane == 0) {
            float* y = a.seg[s].y + row;
            if (NMAT == 2) *y = silu_mul(v[0], v[1]);
            else if (a.epi == RINA_EPI_ADD) *y = *y + v[0];
            else *y = v[0];
        }
    }
}

// ---------------------------------------------------------------------------
// M > 1 (prompt phase): 32x64 output tiles, K stepped by 32; weights are
// dequantized into LDS as fp32 with the same per-element rule as the
// reference dequant, then a plain fp32 FMA tile product.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float deq_elem(const uint8_t* w, int fmt, int64_t n, int k, int K) {
    if (fmt == RINA_QT_Q4_0) {
        const uint8_t* b = w + (n * (K / 32) + k / 32) * 18;
        int i = k & 31;
        int q = (b[2 + (i >> 1)] >> ((i & 1) * 4)) & 0xF;
        return (float)(q - 7) * f16_to_f32(b[0] | (b[1] << 8));
    } else if (fmt == RINA_QT_Q4_0F) {
        const uint8_t* b = w + (n * (K / 32) + k / 32) * 20;
        int i = k & 31;
        int q = (b[4 + (i >> 1)] >> ((i & 1) * 4)) & 0xF;
        float sc;
        __builtin_memcpy(&sc, b, 4);
        return (float)(q - 7) * sc;
    } else if (fmt == RINA_QT_GGML_Q2_K) {
        int64_t e = n * K + k;
        const uint8_t* bd = w + (e >> 8) * 84;
        int inb = (int)(e & 255);
        int page = inb >> 7, pos = inb & 127, l = pos & 31, g = pos >> 5;
        int is = 8 * page + l / 16;
        uint32_t sc = bd[is + 2 * g];
        float dall = f16_to_f32(bd[80] | (bd[81] << 8)), dmin = f16_to_f32(bd[82] | (bd[83] << 8));
        int q = (bd[16 + 32 * page + l] >> (2 * g)) & 3;
        return fmaf(dall * (float)(sc & 0xF), (float)q, -(dmin * (float)(sc >> 4)));
    }
    return ((const float*)w)[n * K + k];
}

struct GemmArgs {
    const uint8_t* w;
    const uint8_t* w2;
    const float* x;
    float* y;
    int M, N, K, fmt, epi;
};

__global__ __launch_bounds__(256) void gemm_tile_kernel(GemmArgs a) {
    __shared__ float xt[32][33];
    __shared__ float wt[2][64][33];
    const int tid = threadIdx.x;
    const int m0 = blockIdx.y * 32, n0 = blockIdx.x * 64;
    const int tm = tid / 16, tn = tid % 16;   // 16 x 16 threads: 2 m x 4 n each
    const int nm = a.w2 ? 2 : 1;
    float acc[2][2][4] = {};
    for (int k0 = 0; k0 < a.K; k0 += 32) {
        for (int i = tid; i < 32 * 32; i += 256) {
            int r = i / 32, c = i % 32;
            int m = m0 + r, k = k0 + c;
            xt[r][c] = (m < a.M && k < a.K) ? a.x[(int64_t)m * a.K + k] : 0.f;
        }
        for (int mat = 0; mat < nm; mat++) {
            const uint8_t* w = mat ? a.w2 : a.w;
            for (int i = tid; i < 64 * 32; i += 256) {
                int r = i / 32, c = i % 32;
                int n = n0 + r, k = k0 + c;
                wt[mat][r][c] = (n < a.N && k < a.K) ? deq_elem(w, a.fmt, n, k, a.K) : 0.f;
            }
        }
        __syncthreads();
        for (int mat = 0; mat < nm; mat++)
            for (int k = 0; k < 32; k++) {
                float xv0 = xt[tm * 2][k], xv1 = xt[tm * 2 + 1][k];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    float wv = wt[mat][tn + 16 * j][k];
                    acc[mat][0][j] = fmaf(xv0, wv, acc[mat][0][j]);
                    acc[mat][1][j] = fmaf(xv1, wv, acc[mat][1][j]);
                }
            }
        __syncthreads();
    }
    for (int i = 0; i < 2; i++)
        for (int j = 0; j < 4; j++) {
            int m = m0 + tm * 2 + i, n = n0 + tn + 16 * j;
            if (m >= a.M || n >= a.N) continue;
            float* y = a.y + (int64_t)m * a.N + n;
            if (nm == 2) *y = silu_mul(acc[0][i][j], acc[1][i][j]);
            else if (a.epi == RINA_EPI_ADD) *y = *y + acc[0][i][j];
            else *y = acc[0][i][j];
        }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

int fmt_of(int qt) {
    switch (qt) {
        case RINA_QT_Q4_0: return FMT_Q4_0;
        case RINA_QT_Q4_0F: return FMT_Q4_0F;
        case RINA_QT_GGML_Q2_K: return FMT_Q2_K;
        default: return -1;
    }
}

template <int FMT, int WPR, int CPL, int NMAT>
int launch_quant(GemvArgs& a, hipStream_t st) {
    int cus = rina_num_cus();
    int grid = a.total_tiles < cus * 4 ? a.total_tiles : cus * 4;
    size_t lds = 2 * (size_t)NMAT * a.slot + (size_t)NMAT * a.R * WPR * 4;
    hipLaunchKernelGGL((gemv_quant_kernel<FMT, WPR, CPL, NMAT>), dim3(grid), dim3(kWG), lds, st, a);
    return hipGetLastError() == hipSuccess ? RINA_OK : RINA_ERR_HIP;
}

template <int FMT, int NMAT>
int dispatch_wpr(GemvArgs& a, int wpr, int cpl, hipStream_t st) {
    if (wpr == 1) return cpl == 1 ? launch_quant<FMT, 1, 1, NMAT>(a, st) : RINA_ERR_SHAPE;
    if (wpr == 2) return cpl == 1 ? launch_quant<FMT, 2, 1, NMAT>(a, st) : RINA_ERR_SHAPE;
    switch (cpl) {
        case 1: return launch_quant<FMT, 4, 1, NMAT>(a, st);
        case 2: return launch_quant<FMT, 4, 2, NMAT>(a, st);
        case 3: return launch_quant<FMT, 4, 3, NMAT>(a, st);
        case 4: return launch_quant<FMT, 4, 4, NMAT>(a, st);
        default: return RINA_ERR_SHAPE;
    }
}

int gemv_quant(const rina_linear_seg* segs, int nseg, int qt, const float* x, int K, int epi, hipStream_t st) {
    int fmt = fmt_of(qt);
    int nmat = (epi == RINA_EPI_SWIGLU) ? 2 : 1;
    int unit = fmt == FMT_Q2_K ? 16 : 32;
    if (K % unit) return RINA_ERR_SHAPE;
    int nunits = K / unit;
    int wpr, cpl;
    if (nunits <= 64) { wpr = 1; cpl = 1; }
    else if (nunits <= 128) { wpr = 2; cpl = 1; }
    else { wpr = 4; cpl = (nunits + 255) / 256; }
    if (cpl > 4) return RINA_ERR_SHAPE;
    int rpi = 4 / wpr;
    GemvArgs a{};
    a.nseg = nseg;
    a.x = x;
    a.K = K;
    a.epi = epi;
    int64_t rowbytes = fmt == FMT_Q4_0 ? (int64_t)(K / 32) * 18 : fmt == FMT_Q4_0F ? (int64_t)(K / 32) * 20 : 0;
    a.rowbytes = (int)rowbytes;
    // LDS bytes of one matrix slot for R rows: the rows' byte range, a
    // 16-byte alignment lead, read slack, and for Q2_K one extra block
    // (a tile's rows may straddle 256-value blocks at both ends).
    auto slot_for = [&](int R) -> int64_t {
        int64_t b = fmt == FMT_Q2_K ? (((int64_t)R * K + 255) / 256 + 1) * 84 : (int64_t)R * rowbytes;
        return (b + 32 + 15) & ~15LL;
    };
    int R = (64 / rpi) * rpi;
    while (R > rpi && slot_for(R) * nmat > kTileBytes) R -= rpi;
    if (slot_for(R) * nmat > kTileBytes) return RINA_ERR_SHAPE;
    int64_t slot_bytes = slot_for(R);
    a.R = R;
    a.slot = (int)slot_bytes;
    int tiles = 0;
    for (int s = 0; s < nseg; s++) {
        a.seg[s].w = (const uint8_t*)segs[s].weight;
        a.seg[s].w2 = (const uint8_t*)segs[s].weight2;
        a.seg[s].y = segs[s].out;
        a.seg[s].N = segs[s].N;
        a.seg[s].tile0 = tiles;
        tiles += (segs[s].N + R - 1) / R;
    }
    a.total_tiles = tiles;
    switch (fmt) {
        case FMT_Q4_0: return nmat == 2 ? dispatch_wpr<FMT_Q4_0, 2>(a, wpr, cpl, st) : dispatch_wpr<FMT_Q4_0, 1>(a, wpr, cpl, st);
        case FMT_Q4_0F: return nmat == 2 ? dispatch_wpr<FMT_Q4_0F, 2>(a, wpr, cpl, st) : dispatch_wpr<FMT_Q4_0F, 1>(a, wpr, cpl, st);
        default: return nmat == 2 ? dispatch_wpr<FMT_Q2_K, 2>(a, wpr, cpl, st) : dispatch_wpr<FMT_Q2_K, 1>(a, wpr, cpl, st);
    }
}

int gemv_f32(const rina_linear_seg* segs, int nseg, const float* x, int K, int epi, hipStream_t st) {
    F32Args a{};
    a.nseg = nseg;
    a.x = x;
    a.K = K;
    a.epi = epi;
    int rows = 0;
    bool vec = (K % 4) == 0;
    for (int s = 0; s < nseg; s++) {
        a.seg[s].w = (const uint8_t*)segs[s].weight;
        a.seg[s].w2 = (const uint8_t*)segs[s].weight2;
        a.seg[s].y = segs[s].out;
        a.seg[s].N = segs[s].N;
        a.seg[s].tile0 = rows;
        rows += segs[s].N;
        vec = vec && ((uintptr_t)segs[s].weight % 16 == 0) && (!segs[s].weight2 || (uintptr_t)segs[s].weight2 % 16 == 0);
    }
    a.total_rows = rows;
    int cus = rina_num_cus();
    int grid = (rows + 3) / 4;
    if (grid > cus * 8) grid = cus * 8;
    size_t lds = (size_t)K * 4;
    if (lds > 64 * 1024) return RINA_ERR_SHAPE;
    bool two = (epi == RINA_EPI_SWIGLU);
    if (two) {
        if (vec) hipLaunchKernelGGL((gemv_f32_kernel<2, true>), dim3(grid), dim3(kWG), lds, st, a);
        else hipLaunchKernelGGL((gemv_f32_kernel<2, false>), dim3(grid), dim3(kWG), lds, st, a);
    } else {
        if (vec) hipLaunchKernelGGL((gemv_f32_kernel<1, true>), dim3(grid), dim3(kWG), lds, st, a);
        else hipLaunchKernelGGL((gemv_f32_kernel<1, false>), dim3(grid), dim3(kWG), lds, st, a);
    }
    return hipGetLastError() == hipSuccess ? RINA_OK : RINA_ERR_HIP;
}

int gemm_tiled(const rina_linear_seg& seg, int qt, const float* x, int M, int K, int epi, hipStream_t st) {
    GemmArgs a{(const uint8_t*)seg.weight, epi == RINA_EPI_SWIGLU ? (const uint8_t*)seg.weight2 : nullptr,
               x, seg.out, M, seg.N, K, qt, epi};
    dim3 grid((seg.N + 63) / 64, (M + 31) / 32);
    hipLaunchKernelGGL(gemm_tile_kernel, grid, dim3(256), 0, st, a);
    return hipGetLastError() == hipSuccess ? RINA_OK : RINA_ERR_HIP;
}

bool qt_supported(int qt) {
    return qt == RINA_QT_Q4_0 || qt == RINA_QT_Q4_0F || qt == RINA_QT_GGML_Q2_K || qt == RINA_QT_FP32;
}

}  // namespace

extern "C" int rina_hip_linear_fused(const rina_linear_seg* segs, int nseg, int qt, const float* input,
                                     int M, int K, int epi, void* stream) {
    if (!segs || nseg < 1 || nseg > 3 || !input || M < 1 || K < 1) return RINA_ERR_ARG;
    if (!qt_supported(qt)) return RINA_ERR_QTYPE;
    if (epi < RINA_EPI_STORE || epi > RINA_EPI_SWIGLU) return RINA_ERR_ARG;
    if (epi == RINA_EPI_SWIGLU && nseg != 1) return RINA_ERR_ARG;
    if ((qt == RINA_QT_Q4_0 || qt == RINA_QT_Q4_0F) && (K % 32)) return RINA_ERR_SHAPE;
    for (int s = 0; s < nseg; s++) {
        if (!segs[s].weight || !segs[s].out || segs[s].N < 1) return RINA_ERR_ARG;
        if (epi == RINA_EPI_SWIGLU && !segs[s].weight2) return RINA_ERR_ARG;
        if ((uintptr_t)segs[s].weight % 4 || (segs[s].weight2 && (uintptr_t)segs[s].weight2 % 4)) return RINA_ERR_ARG;
    }
    hipStream_t st = as_stream(stream);
    if (M > 1) {
        for (int s = 0; s < nseg; s++) {
            int rc = gemm_tiled(segs[s], qt, input, M, K, epi, st);
            if (rc) return rc;
        }
        return RINA_OK;
    }
    if (qt == RINA_QT_FP32) return gemv_f32(segs, nseg, input, K, epi, st);
    if ((uintptr_t)input % 16) {   // register staging of x uses 16-byte loads
        for (int s = 0; s < nseg; s++) {
            int rc = gemm_tiled(segs[s], qt, input, M, K, epi, st);
            if (rc) return rc;
        }
        return RINA_OK;
    }
    return gemv_quant(segs, nseg, qt, input, K, epi, st);
}

extern "C" int rina_hip_linear(const void* weight, int qt, const float* input, float* output, int M, int N, int K,
                               void* stream) {
    if (!weight || !input || !output || M < 1 || N < 1 || K < 1) return RINA_ERR_ARG;
    if (!qt_supported(qt)) return RINA_ERR_QTYPE;
    hipStream_t st = as_stream(stream);
    // Out-of-place semantics for input == output (or overlapping ranges):
    // compute into library scratch, then copy (stream-ordered, no sync).
    const char* ib = (const char*)input;
    const char* ie = ib + (size_t)M * K * 4;
    const char* ob = (const char*)output;
    const char* oe = ob + (size_t)M * N * 4;
    bool alias = ib < oe && ob < ie;
    float* dst = output;
    if (alias) {
        dst = (float*)rina_scratch((size_t)M * N * 4);
        if (!dst) return RINA_ERR_HIP;
    }
    rina_linear_seg seg{weight, nullptr, dst, N};
    int rc = rina_hip_linear_fused(&seg, 1, qt, input, M, K, RINA_EPI_STORE, stream);
    if (rc) return rc;
    if (alias && hipMemcpyAsync(output, dst, (size_t)M * N * 4, hipMemcpyDeviceToDevice, st) != hipSuccess)
        return RINA_ERR_HIP;
    return RINA_OK;
}
