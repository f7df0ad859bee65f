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
#include <type_traits>
#include "rina_common.hpp"
#include "q2k_col.hpp"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWG = 256;
constexpr int kMaxChunks = 4;              // 16-byte chunks per thread per tile
constexpr int kTileBytes = kWG * kMaxChunks * 16;   // 16 KiB per tile (all matrices)


struct GemvSeg {
    const uint8_t* w;
    const uint8_t* w2;
    float* y;
    int N;
    int tile0;
};

constexpr int kMaxDirectSegs = 6;   // row segments of one direct-kernel launch (tile kernel: 3)

struct GemvArgs {
    GemvSeg seg[3];
    GemvSeg seg_hi[3];   // segments 3..5 (direct kernel only, read with constant indices)
    int nseg;
    float* xn;           // direct kernel with a norm prologue: workgroup 0 stores the normalized row (or NULL)
    const float* x;
    int K;
    int R;            // rows per tile
    int total_tiles;
    int epi;
    int rowbytes;     // Q4 formats: bytes per row
    int slot;         // LDS bytes per matrix slot (16-byte multiple)
    const float* nw;  // prologue norm weight
    float eps;
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

// Thread tid loads chunks tid + k*kWG (k < kMaxChunks/NMAT) of each matrix's
// 16-byte-aligned byte window; the chunk -> matrix mapping is static.
template <int FMT, int NMAT>
__device__ __forceinline__ void tile_windows(const GemvArgs& a, int t, const uint8_t* (&base)[2], int (&nch)[2]) {
    int s, n0, rows;
    tile_of(a, t, s, n0, rows);
    int64_t start, len;
    tile_bytes<FMT>(a, n0, rows, start, len);
#pragma unroll
    for (int m = 0; m < NMAT; m++) {
        const uint8_t* g = (m == 0 ? a.seg[s].w : a.seg[s].w2) + start;
        int lead = (int)((uintptr_t)g & 15);
        base[m] = g - lead;
        nch[m] = (int)((lead + len + 15) >> 4);
    }
}

template <int FMT, int NMAT>
__device__ __forceinline__ void tile_load(const GemvArgs& a, int t, u32x4 (&pre)[kMaxChunks]) {
    constexpr int CPM = kMaxChunks / NMAT;
    const uint8_t* base[2];
    int nch[2];
    tile_windows<FMT, NMAT>(a, t, base, nch);
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < kMaxChunks; i++) {
        const int m = i / CPM, c = tid + (i % CPM) * kWG;
        if (c < nch[m]) pre[i] = gld_nt((const u32x4*)(base[m]) + c);
    }
}

template <int FMT, int NMAT>
__device__ __forceinline__ void tile_store(const GemvArgs& a, int t, const u32x4 (&pre)[kMaxChunks], uint8_t* buf) {
    constexpr int CPM = kMaxChunks / NMAT;
    const uint8_t* base[2];
    int nch[2];
    tile_windows<FMT, NMAT>(a, t, base, nch);
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < kMaxChunks; i++) {
        const int m = i / CPM, c = tid + (i % CPM) * kWG;
        if (c < nch[m]) *(u32x4*)(buf + m * a.slot + c * 16) = pre[i];
    }
}

__device__ __forceinline__ uint32_t lds_u32(const uint8_t* p) { return *(const uint32_t*)p; }
__device__ __forceinline__ uint32_t lds_u16(const uint8_t* p) { return *(const uint16_t*)p; }

// exact integer sum_i q_i X_i of one 16-value Q2_K unit (qs bytes q[0..3], shift 2g), as float
template <int CPL>
__device__ __forceinline__ float q2_dot(const uint32_t (&q)[4], uint32_t sh, const XCols<FMT_Q2_K, CPL>& xc, int j) {
    int a0 = 0, a1 = 0, a2 = 0;
#pragma unroll
    for (int d = 0; d < 4; d++) {
        const int t = (int)and_opaque(q[d] >> sh, 0x03030303u);
        a0 = __builtin_amdgcn_sdot4(t, xc.dg[j][0][d], a0, false);
        a1 = __builtin_amdgcn_sdot4(t, xc.dg[j][1][d], a1, false);
        a2 = __builtin_amdgcn_sdot4(t, xc.dg[j][2][d], a2, false);
    }
    return fmaf(65536.0f, (float)a2, fmaf(256.0f, (float)a1, (float)a0));
}


template <int NMAT>
__device__ __forceinline__ void epilogue(const GemvArgs& a, int s, int n, const float (&v)[2]) {
    float* y = a.seg[s].y + n;
    if (NMAT == 2) gst(y, silu_mul(v[0], v[1]));
    else if (a.epi == RINA_EPI_ADD) gst(y, gld(y) + v[0]);
    else gst(y, v[0]);
}

// One tile of R rows from LDS: lane owns units (cp*CPL+j)*64+lane of each row.
template <int FMT, int WPR, int CPL, int NMAT>
__device__ __forceinline__ void compute_tile(const GemvArgs& a, int t, const uint8_t* buf, const uint8_t* smem,
                                             const XCols<FMT, CPL>& xc, float* red) {
    constexpr int UNIT = (FMT == FMT_Q2_K) ? 16 : 32;
    constexpr int RPI = 4 / WPR;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int rs = wave / WPR, cp = wave % WPR;
    const int K = a.K;
    const int nunits = K / UNIT;
    int s, n0, rows;
    tile_of(a, t, s, n0, rows);
    int64_t start, len;
    tile_bytes<FMT>(a, n0, rows, start, len);
    int lead[2];
#pragma unroll
    for (int m = 0; m < NMAT; m++) lead[m] = (int)((uintptr_t)((m == 0 ? a.seg[s].w : a.seg[s].w2) + start) & 15);

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
                if constexpr (FMT == FMT_Q4_0F) {
                    const uint8_t* bp = sl + r * a.rowbytes + u * 20;
                    float sc = __uint_as_float(lds_u32(bp));
                    uint32_t nib[4];
#pragma unroll
                    for (int d = 0; d < 4; d++) nib[d] = lds_u32(bp + 4 + 4 * d);
                    part = fmaf(sc * xc.xe[j], q4_dot(nib, xc, j), part);
                } else if constexpr (FMT == FMT_Q4_0) {
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
                    part = fmaf(sc * xc.xe[j], q4_dot(nib, xc, j), part);
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
                    float dl = dall * (float)(scb & 0xF), ml = dmin * (float)(scb >> 4);
                    part = fmaf(dl * xc.xe[j], q2_dot(q, 2u * g, xc, j), fmaf(-ml, xc.xs[j], part));
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

// Lane-owned activation columns (and prologue norm weights), raw.
template <int FMT, int WPR, int CPL, int PRO>
struct XRaw {
    static constexpr int UNIT = (FMT == FMT_Q2_K) ? 16 : 32;
    float x[CPL][UNIT];
    float w[PRO != RINA_PRO_NONE ? CPL : 1][PRO != RINA_PRO_NONE ? UNIT : 1];
};

template <int FMT, int WPR, int CPL, int PRO>
__device__ __forceinline__ void load_x_raw(const GemvArgs& a, XRaw<FMT, WPR, CPL, PRO>& r) {
    constexpr int UNIT = XRaw<FMT, WPR, CPL, PRO>::UNIT;
    const int lane = threadIdx.x & 63, cp = (threadIdx.x >> 6) % WPR;
    const int nunits = a.K / UNIT;
#pragma unroll
    for (int j = 0; j < CPL; j++) {
        int u = (cp * CPL + j) * 64 + lane;
        if (u < nunits) {
            const f32x4* xp = (const f32x4*)(a.x + (int64_t)u * UNIT);
#pragma unroll
            for (int i = 0; i < UNIT / 4; i++) {
                f32x4 v = gld(xp + i);
                r.x[j][4 * i + 0] = v.x; r.x[j][4 * i + 1] = v.y;
                r.x[j][4 * i + 2] = v.z; r.x[j][4 * i + 3] = v.w;
            }
            if constexpr (PRO != RINA_PRO_NONE) {
                const f32x4* wp = (const f32x4*)(a.nw + (int64_t)u * UNIT);
#pragma unroll
                for (int i = 0; i < UNIT / 4; i++) {
                    f32x4 v = gld(wp + i);
                    r.w[j][4 * i + 0] = v.x; r.w[j][4 * i + 1] = v.y;
                    r.w[j][4 * i + 2] = v.z; r.w[j][4 * i + 3] = v.w;
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < UNIT; i++) r.x[j][i] = 0.f;
            if constexpr (PRO != RINA_PRO_NONE) {
#pragma unroll
                for (int i = 0; i < UNIT; i++) r.w[j][i] = 0.f;
            }
        }
    }
}

// Normalize (PRO: 0 none, 1 RMSNorm, 2 LayerNorm; needs WPR == 1 so every
// wave holds the whole row) and digitize the lane's columns.
template <int FMT, int WPR, int CPL, int PRO>
__device__ __forceinline__ void prep_x(const GemvArgs& a, XRaw<FMT, WPR, CPL, PRO>& r, XCols<FMT, CPL>& xc) {
    constexpr int UNIT = XRaw<FMT, WPR, CPL, PRO>::UNIT;
    if constexpr (PRO != RINA_PRO_NONE) {
        const int lane = threadIdx.x & 63, cp = (threadIdx.x >> 6) % WPR;
        const int nunits = a.K / UNIT;
        const float d = (float)a.K;
        float mean = 0.f;
        if (PRO == RINA_PRO_LAYERNORM) {
            float sm = 0.f;
#pragma unroll
            for (int j = 0; j < CPL; j++)
#pragma unroll
                for (int i = 0; i < UNIT; i++) sm += r.x[j][i];
            mean = wave_sum(sm) / d;
        }
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < CPL; j++) {
            int u = (cp * CPL + j) * 64 + lane;
            if (u >= nunits) continue;
#pragma unroll
            for (int i = 0; i < UNIT; i++) {
                float t = r.x[j][i] - mean;
                ss = fmaf(t, t, ss);
            }
        }
        const float inv = 1.0f / sqrtf(wave_sum(ss) / d + a.eps);
#pragma unroll
        for (int j = 0; j < CPL; j++)
#pragma unroll
            for (int i = 0; i < UNIT; i++) r.x[j][i] = (r.x[j][i] - mean) * inv * r.w[j][i];
    }
#pragma unroll
    for (int j = 0; j < CPL; j++) digitize<FMT, CPL>(xc, j, r.x[j]);
}

template <int FMT, int WPR, int CPL, int PRO>
__device__ __forceinline__ void load_x(const GemvArgs& a, XCols<FMT, CPL>& xc) {
    XRaw<FMT, WPR, CPL, PRO> r;
    load_x_raw<FMT, WPR, CPL, PRO>(a, r);
    prep_x<FMT, WPR, CPL, PRO>(a, r, xc);
}

// Tiles are dealt round-robin to the workgroups; two tiles ahead are kept in
// flight in registers (sets A and B) while the LDS copy of the current one is
// consumed, and the first loads go out before the activation vector is read.
template <int FMT, int WPR, int CPL, int NMAT, int PRO>
__global__ __launch_bounds__(kWG) void gemv_quant_kernel(GemvArgs a) {
    constexpr int UNIT = (FMT == FMT_Q2_K) ? 16 : 32;
    extern __shared__ __align__(16) uint8_t smem[];
    const int T = a.total_tiles, G = gridDim.x;
    const int bufbytes = NMAT * a.slot;
    uint8_t* buf0 = smem;
    uint8_t* buf1 = smem + bufbytes;
    float* red = (float*)(smem + 2 * bufbytes);   // [NMAT][R][WPR]

    u32x4 pA[kMaxChunks], pB[kMaxChunks];
    int t = blockIdx.x;
    if (t < T) tile_load<FMT, NMAT>(a, t, pA);
    if (t + G < T) tile_load<FMT, NMAT>(a, t + G, pB);

    XCols<FMT, CPL> xc;
    load_x<FMT, WPR, CPL, PRO>(a, xc);

    for (; t < T; t += 2 * G) {
        tile_store<FMT, NMAT>(a, t, pA, buf0);
        __syncthreads();
        if (t + 2 * G < T) tile_load<FMT, NMAT>(a, t + 2 * G, pA);
        compute_tile<FMT, WPR, CPL, NMAT>(a, t, buf0, smem, xc, red);
        if (t + G >= T) break;
        tile_store<FMT, NMAT>(a, t + G, pB, buf1);
        __syncthreads();
        if (t + 3 * G < T) tile_load<FMT, NMAT>(a, t + 3 * G, pB);
        compute_tile<FMT, WPR, CPL, NMAT>(a, t + G, buf1, smem, xc, red);
    }
}

// ---------------------------------------------------------------------------
// Direct-load Q4 matvec (M = 1).  Lane l owns block column cp*64+l of every
// row; a wave takes RB rows at a time and loads each of its blocks straight
// from HBM (one 16-byte + one 4-byte load per block at 4-byte alignment, the
// 18/20-byte block layout needs no staging), so every lane keeps RB*NMAT
// blocks in flight and the RB*NMAT row sums reduce as independent DPP
// chains.  No LDS and no barrier unless a row spans several waves (WPR > 1,
// one LDS exchange per row group).
// ---------------------------------------------------------------------------


// Blocks of one row group held in registers: RB rows x NMAT matrices.
template <int RB>
struct DirectBlk {
    float sc[RB][2];
    uint32_t nib[RB][2][4];
    int seg[RB], row[RB];
    bool ok[RB];
    float yres[RB];     // one matrix: y of the group's rows (lane 0 finishes them, one wave per row)
    float yep;          // one matrix, 2-4 waves per row: y of the row this thread finishes
};

// Q2_K in the direct kernel: a lane's column is 32 consecutive values of a
// row, which in the 256-value block layout (ops/linear.cu:322-338) is shift
// group g of one 128-value page: the page's 32 qs bytes (2 bits per value at
// bit 2g of byte i for value i of each 16-value half), the two half scale
// bytes (sc | m << 4) and the block's fp16 d, dmin.  32-value columns never
// straddle a block because row starts are multiples of 32 values.
template <int RB>
struct DirectBlkQ2 {
    // 4+ rows per wave: quad form (this lane's quarter of the half page's qs
    // bytes, exchanged at use); 1-2 rows: the whole 32 bytes per lane, since
    // with so few loads in flight the exchange's latency costs more than the
    // repeated bytes (W_o 2048 x 2048: 3.7 vs 4.4 us)
    static constexpr bool QUAD = RB >= 4;
    uint32_t qs[RB][2][QUAD ? 2 : 8];
    uint32_t sm[RB][2];     // dword holding the scale bytes of halves 0 and 1 (q2_sm16)
    uint32_t dd[RB][2];     // d | dmin << 16
    int sh[RB];             // 2g
    int seg[RB], row[RB];
    bool ok[RB];
    float yres[RB];         // as DirectBlk
    float yep;
};

template <int FMT, int RB>
using DirectBlkT = typename std::conditional<FMT == FMT_Q2_K, DirectBlkQ2<RB>, DirectBlk<RB>>::type;

__device__ __forceinline__ uint64_t uni64(const void* p) {
    const uint64_t v = (uint64_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return ((uint64_t)hi << 32) | lo;
}

// Segment table as wave-uniform values read once at kernel entry.  A field
// of segment sg is picked with integer arithmetic on these values: indexing
// the argument struct (or any array) with a run-time segment number makes
// the compiler copy it to scratch memory.
template <int NS>
struct DirectSegs {
    uint64_t w[NS], v[NS], y[NS];
    int t[NS];
    int nseg;
    __device__ __forceinline__ explicit DirectSegs(const GemvArgs& a) {
#pragma unroll
        for (int i = 0; i < NS; i++) {
            const GemvSeg& g = i < 3 ? a.seg[i] : a.seg_hi[i - 3];
            w[i] = uni64(g.w);
            v[i] = uni64(g.w2);
            y[i] = uni64(g.y);
            t[i] = __builtin_amdgcn_readfirstlane(g.tile0);
        }
        nseg = __builtin_amdgcn_readfirstlane(a.nseg);
    }
    // segments are in row order: the segment of virtual row vr
    __device__ __forceinline__ int seg_of(int vr) const {
        int s = 0;
#pragma unroll
        for (int i = 1; i < NS; i++) s += (i < nseg && vr >= t[i]) ? 1 : 0;
        return s;
    }
    __device__ __forceinline__ static uint64_t sel(int sg, const uint64_t (&f)[NS]) {
        uint64_t r = 0;
#pragma unroll
        for (int i = 0; i < NS; i++) r |= f[i] & ((uint64_t)0 - (uint64_t)(sg == i));
        return r;
    }
    __device__ __forceinline__ int t0(int sg) const {
        int r = 0;
#pragma unroll
        for (int i = 0; i < NS; i++) r |= t[i] & -(int)(sg == i);
        return r;
    }
    __device__ __forceinline__ const uint8_t* wt(int sg, int m) const {
        return (const uint8_t*)(m == 0 ? sel(sg, w) : sel(sg, v));
    }
    __device__ __forceinline__ float* out(int sg) const { return (float*)sel(sg, y); }
};

// Issue the loads of row group grp (virtual rows grp*RB ..) for block column u.
template <int FMT, int NMAT, int RB, typename Segs>
__device__ __forceinline__ void direct_issue(const GemvArgs& a, const Segs& S, int grp, int u, bool active,
                                             DirectBlk<RB>& b) {
    constexpr int BB = FMT == FMT_Q4_0F ? 20 : 18;
#pragma unroll
    for (int i = 0; i < RB; i++) {
        const int vr = grp * RB + i;
        const int sg = S.seg_of(vr);
        b.seg[i] = sg;
        b.row[i] = (grp < a.total_tiles && vr < a.R) ? vr - S.t0(sg) : -1;
        // Loads are unconditional (a branch around them costs the waitcnt
        // pass its count and it then waits for every load): lanes past the
        // row's end or rows past the matrix read block 0 of the segment and
        // get scale 0.
        const bool ok = active && b.row[i] >= 0;
        const int64_t off = ok ? (int64_t)b.row[i] * a.rowbytes + (int64_t)u * BB : 0;
#pragma unroll
        for (int m = 0; m < NMAT; m++) load_q4_block<FMT>(S.wt(sg, m) + off, b.sc[i][m], b.nib[i][m]);
        b.ok[i] = ok;   // applied where the scale is used, so nothing waits here
    }
}

// Q2_K: column u of row n is flat elements [nK + 32u, nK + 32u + 32).
template <int FMT, int NMAT, int RB, typename Segs>
__device__ __forceinline__ void direct_issue(const GemvArgs& a, const Segs& S, int grp, int u, bool active,
                                             DirectBlkQ2<RB>& b) {
#pragma unroll
    for (int i = 0; i < RB; i++) {
        const int vr = grp * RB + i;
        const int sg = S.seg_of(vr);
        b.seg[i] = sg;
        b.row[i] = (grp < a.total_tiles && vr < a.R) ? vr - S.t0(sg) : -1;
        const bool ok = active && b.row[i] >= 0;
        const int64_t e = ok ? (int64_t)b.row[i] * a.K + 32 * u : 0;
        const int64_t off = (e >> 8) * 84;
        const int page = (int)(e >> 7) & 1, g = (int)(e >> 5) & 3;
        b.sh[i] = 2 * g;
#pragma unroll
        for (int m = 0; m < NMAT; m++) {
            if constexpr (DirectBlkQ2<RB>::QUAD) {
                Q2ColQ c;
                q2_colq_load(S.wt(sg, m) + off, page, g, c);
                b.qs[i][m][0] = c.q[0]; b.qs[i][m][1] = c.q[1];
                b.sm[i][m] = c.sm;
                b.dd[i][m] = c.dd;
            } else {
                Q2Col c;
                q2_col_load(S.wt(sg, m) + off, page, g, c);
#pragma unroll
                for (int z = 0; z < 8; z++) b.qs[i][m][z] = c.qs[z];
                b.sm[i][m] = c.sm;
                b.dd[i][m] = c.dd;
            }
        }
        b.ok[i] = ok;
    }
}

// The output words a one-matrix launch's epilogue finishes, loaded with the
// weights of their row group instead of after the row sums: the residual
// add then costs no memory round trip at the end of the launch.  Every lane
// loads (the finishing lanes use theirs; rows past the end read row 0 of
// their segment), so the load counters stay exact.  Each output word is read
// and written by one thread only, and never by another workgroup.
template <int WPR, int NMAT, int RB, typename Segs, typename Blk>
__device__ __forceinline__ void direct_yload(const GemvArgs& a, const Segs& S, int it, Blk& b) {
    if constexpr (NMAT == 1) {
        if constexpr (WPR == 1) {
#pragma unroll
            for (int i = 0; i < RB; i++) b.yres[i] = gld(S.out(b.seg[i]) + (b.row[i] >= 0 ? b.row[i] : 0));
        } else {
            constexpr int RPI = 4 / WPR;
            const int tid = threadIdx.x;
            const int k = tid < RPI * RB ? tid : 0;
            const int grp = it * RPI + k / RB, vr = grp * RB + k % RB;
            const bool ok = grp < a.total_tiles && vr < a.R;
            const int sg = S.seg_of(ok ? vr : 0);
            b.yep = gld(S.out(sg) + (ok ? vr - S.t0(sg) : 0));
        }
    }
}

template <int NMAT, bool YL, typename Segs>
__device__ __forceinline__ void direct_epilogue(const GemvArgs& a, const Segs& S, int sg, int n,
                                                const float (&v)[2], float yold) {
    float* y = S.out(sg) + n;
    if (NMAT == 2) gst(y, silu_mul(v[0], v[1]));
    else if (YL) gst(y, yold + v[0]);                   // YL: exactly the residual epilogue
    else if (a.epi == RINA_EPI_ADD) gst(y, gld(y) + v[0]);
    else gst(y, v[0]);
}

// Row sums of one row group and their epilogue.
template <int FMT, int WPR, int NMAT, int RB, bool YL, typename Segs>
__device__ __forceinline__ void direct_consume(const GemvArgs& a, const Segs& S, const DCols<FMT>& xc,
                                               const DirectBlkT<FMT, RB>& cur, int it, int rs, int cp,
                                               float (*red)[RB * NMAT][WPR]) {
    constexpr int RPI = 4 / WPR;
    const int tid = threadIdx.x, lane = tid & 63;
    float part[RB][2];
#pragma unroll
    for (int i = 0; i < RB; i++)
#pragma unroll
        for (int m = 0; m < NMAT; m++) {
            if constexpr (FMT == FMT_Q2_K) {
                Q2Col c;
                if constexpr (DirectBlkQ2<RB>::QUAD) {
                    // the quad exchange runs on every lane, outside the row test
                    const Q2ColQ cq{{cur.qs[i][m][0], cur.qs[i][m][1]}, 0u, 0u, 0u};
                    q2_colq_expand(cq, c);
                } else {
#pragma unroll
                    for (int z = 0; z < 8; z++) c.qs[z] = cur.qs[i][m][z];
                }
                part[i][m] = wave_sum(cur.ok[i] ? q2_col(c.qs, q2_sm16(cur.sm[i][m], cur.sh[i]), cur.dd[i][m], cur.sh[i], xc) : 0.f);
            }
            else
                part[i][m] = wave_sum((cur.ok[i] ? cur.sc[i][m] : 0.f) * xc.xe[0] * q4_dot(cur.nib[i][m], xc, 0));
        }
    if (WPR == 1) {
        if (lane == 0) {
#pragma unroll
            for (int i = 0; i < RB; i++)
                if (cur.row[i] >= 0) {
                    float v[2] = {part[i][0], NMAT == 2 ? part[i][1] : 0.f};
                    direct_epilogue<NMAT, YL>(a, S, cur.seg[i], cur.row[i], v, YL ? cur.yres[i] : 0.f);
                }
        }
    } else {
        if (lane == 0) {
#pragma unroll
            for (int i = 0; i < RB; i++)
#pragma unroll
                for (int m = 0; m < NMAT; m++) red[rs][i * NMAT + m][cp] = part[i][m];
        }
        __syncthreads();
        if (tid < RPI * RB) {
            const int r2 = tid / RB, i = tid % RB;
            const int grp = it * RPI + r2, vr = grp * RB + i;
            if (grp < a.total_tiles && vr < a.R) {
                const int sg = S.seg_of(vr);
                float v[2] = {0.f, 0.f};
#pragma unroll
                for (int m = 0; m < NMAT; m++)
#pragma unroll
                    for (int c = 0; c < WPR; c++) v[m] += red[r2][i * NMAT + m][c];
                direct_epilogue<NMAT, YL>(a, S, sg, vr - S.t0(sg), v, YL ? cur.yep : 0.f);
            }
        }
        __syncthreads();
    }
}

// GemvArgs reuse for this kernel: total_tiles = number of row groups,
// R = number of virtual rows, seg[s].tile0 = first virtual row of segment s.
// ITERS == 1: one iteration per workgroup (the grid covers every row
// group), straight-line code.  ITERS == 0: iterations alternate between two
// register sets (A, B), the next group's loads issued before the current
// group is reduced; each path has its own straight-line code so the load
// counters stay exact.  YL: residual epilogue, the old output words loaded
// with each group's weights.
template <int FMT, int WPR, int NMAT, int PRO, int RB, int NS, int ITERS, bool YL>
__global__ __launch_bounds__(kWG) void gemv_direct_kernel(GemvArgs a) {
    constexpr int RPI = 4 / WPR;                 // row groups per workgroup iteration
    __shared__ float red[RPI][RB * NMAT][WPR];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rs = wave / WPR, cp = wave % WPR;
    const int u = cp * 64 + lane;                // this lane's block column
    const bool active = u < a.K / 32;
    const int G = gridDim.x;
    const int ngrp = a.total_tiles;
    const DirectSegs<NS> S(a);

    // activation loads, then the first row group's weight loads, then the
    // activation prep (overlapping the weight loads)
    constexpr int TPC = WPR == 1 ? 4 : WPR == 2 ? 2 : 1;
    PrepRaw<TPC, PRO> raw;
    const PrepSrc src{a.x, a.nw, a.K, a.eps, a.xn};
    wg_prep_load<TPC, PRO>(src, raw);
    auto prep_cols = [&](DCols<FMT>& xc) {
        if constexpr (WPR == 4) {
            // u == threadIdx.x: every thread prepares its own column
            __shared__ float red[8];
            own_prep_x<FMT, PRO>(src, raw, red, xc);
        } else {
            __shared__ PrepLds prep;
            wg_prep_x<FMT, TPC, PRO>(src, raw, prep);
            read_cols<FMT>(prep, u, active, xc);
        }
    };
    if constexpr (ITERS == 1) {
        DirectBlkT<FMT, RB> A;
        direct_issue<FMT, NMAT, RB>(a, S, blockIdx.x * RPI + rs, u, active, A);
        if constexpr (YL) direct_yload<WPR, NMAT, RB>(a, S, blockIdx.x, A);
        DCols<FMT> xc;
        prep_cols(xc);
        direct_consume<FMT, WPR, NMAT, RB, YL>(a, S, xc, A, blockIdx.x, rs, cp, red);
    } else {
        int it = blockIdx.x;
        DirectBlkT<FMT, RB> A, B;
        direct_issue<FMT, NMAT, RB>(a, S, it * RPI + rs, u, active, A);
        if constexpr (YL) direct_yload<WPR, NMAT, RB>(a, S, it, A);
        DCols<FMT> xc;
        prep_cols(xc);

        for (;;) {
            if ((it + G) * RPI < ngrp) {
                direct_issue<FMT, NMAT, RB>(a, S, (it + G) * RPI + rs, u, active, B);
                if constexpr (YL) direct_yload<WPR, NMAT, RB>(a, S, it + G, B);
                direct_consume<FMT, WPR, NMAT, RB, YL>(a, S, xc, A, it, rs, cp, red);
            } else {
                direct_consume<FMT, WPR, NMAT, RB, YL>(a, S, xc, A, it, rs, cp, red);
                break;
            }
            it += G;
            if ((it + G) * RPI < ngrp) {
                direct_issue<FMT, NMAT, RB>(a, S, (it + G) * RPI + rs, u, active, A);
                if constexpr (YL) direct_yload<WPR, NMAT, RB>(a, S, it + G, A);
                direct_consume<FMT, WPR, NMAT, RB, YL>(a, S, xc, B, it, rs, cp, red);
            } else {
                direct_consume<FMT, WPR, NMAT, RB, YL>(a, S, xc, B, it, rs, cp, red);
                break;
            }
            it += G;
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
    int pro;
    const float* nw;
    float eps;
    unsigned long long* keys;   // argmax epilogue: one key per workgroup (one segment, store epilogue)
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
            f32x4 a0 = gld_nt(w4 + k);
            f32x4 a1 = gld_nt(w4 + k + 64);
            f32x4 a2 = gld_nt(w4 + k + 128);
            f32x4 a3 = gld_nt(w4 + k + 192);
            f32x4 b0 = x4[k], b1 = x4[k + 64], b2 = x4[k + 128], b3 = x4[k + 192];
            s0 = fmaf(b0.x, a0.x, s0); s0 = fmaf(b0.y, a0.y, s0); s0 = fmaf(b0.z, a0.z, s0); s0 = fmaf(b0.w, a0.w, s0);
            s1 = fmaf(b1.x, a1.x, s1); s1 = fmaf(b1.y, a1.y, s1); s1 = fmaf(b1.z, a1.z, s1); s1 = fmaf(b1.w, a1.w, s1);
            s2 = fmaf(b2.x, a2.x, s2); s2 = fmaf(b2.y, a2.y, s2); s2 = fmaf(b2.z, a2.z, s2); s2 = fmaf(b2.w, a2.w, s2);
            s3 = fmaf(b3.x, a3.x, s3); s3 = fmaf(b3.y, a3.y, s3); s3 = fmaf(b3.z, a3.z, s3); s3 = fmaf(b3.w, a3.w, s3);
        }
        for (; k < n4; k += 64) {
            f32x4 a0 = gld_nt(w4 + k);
            f32x4 b0 = x4[k];
            s0 = fmaf(b0.x, a0.x, s0); s0 = fmaf(b0.y, a0.y, s0); s0 = fmaf(b0.z, a0.z, s0); s0 = fmaf(b0.w, a0.w, s0);
        }
    } else {
        for (int k = lane; k < K; k += 64) s0 = fmaf(xl[k], gld(w + k), s0);
    }
    return (s0 + s1) + (s2 + s3);
}

// Rows of K <= 2048 values: a wave takes RPW rows at a time and issues all
// their 16-byte loads (NV per lane per row, lane + 64 t) before any
// arithmetic, so a lane keeps RPW * NV loads in flight.
template <int NMAT, int NV>
__device__ __forceinline__ void f32_rows_short(const F32Args& a, const float* xs_lds, int gw, int nw,
                                               unsigned long long& best) {
    constexpr int RPW = NMAT == 2 ? 2 : 4;
    const int lane = threadIdx.x & 63;
    const int K = a.K, n4 = K >> 2;
    const f32x4* x4 = (const f32x4*)xs_lds;
    for (int r0 = gw * RPW; r0 < a.total_rows; r0 += nw * RPW) {
        f32x4 w[RPW][NMAT][NV];
        int seg[RPW], row[RPW];
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            const int vr = min(r0 + r, a.total_rows - 1);
            int s = 0;
            if (a.nseg > 1 && vr >= a.seg[1].tile0) s = 1;
            if (a.nseg > 2 && vr >= a.seg[2].tile0) s = 2;
            seg[r] = s;
            row[r] = vr - a.seg[s].tile0;
#pragma unroll
            for (int m = 0; m < NMAT; m++) {
                const f32x4* wr = (const f32x4*)(m == 0 ? a.seg[s].w : a.seg[s].w2) + (int64_t)row[r] * n4;
#pragma unroll
                for (int t = 0; t < NV; t++) {
                    const int k = lane + 64 * t;
                    w[r][m][t] = gld_nt(wr + (k < n4 ? k : 0));
                }
            }
        }
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            float v[2];
#pragma unroll
            for (int m = 0; m < NMAT; m++) {
                float s0 = 0.f, s1 = 0.f;
#pragma unroll
                for (int t = 0; t < NV; t++) {
                    const int k = lane + 64 * t;
                    const f32x4 b = k < n4 ? x4[k] : f32x4{0.f, 0.f, 0.f, 0.f};
                    float& acc = (t & 1) ? s1 : s0;
                    acc = fmaf(b.x, w[r][m][t].x, acc); acc = fmaf(b.y, w[r][m][t].y, acc);
                    acc = fmaf(b.z, w[r][m][t].z, acc); acc = fmaf(b.w, w[r][m][t].w, acc);
                }
                v[m] = wave_sum(s0 + s1);
            }
            if (lane == 0 && r0 + r < a.total_rows) {
                float* y = a.seg[seg[r]].y + row[r];
                if (NMAT == 2) gst(y, silu_mul(v[0], v[1]));
                else if (a.epi == RINA_EPI_ADD) gst(y, gld(y) + v[0]);
                else gst(y, v[0]);
                best = umax64(best, argmax_cand(v[0], row[r]));
            }
        }
    }
}

// Rows of K = 128 NV values (K/4 a multiple of 32, not of 64: K = 640 is the
// Jamba LM head): each half wave takes a row, so a lane's NV 16-byte loads
// per row are all in use.  A wave takes 2 * RP rows at a time, all loads
// issued first; the half-wave sums come from lanes 31 and 63 after the
// row_bcast step of the wave reduction.
template <int NMAT, int NV, int RP>
__device__ __forceinline__ void f32_rows_half(const F32Args& a, const float* xs_lds, int gw, int nw,
                                              unsigned long long& best) {
    constexpr int RPW = 2 * RP;
    const int lane = threadIdx.x & 63, hl = lane & 31, half = lane >> 5;
    const int n4 = a.K >> 2;
    const f32x4* x4 = (const f32x4*)xs_lds;
    f32x4 xv[NV];
#pragma unroll
    for (int t = 0; t < NV; t++) xv[t] = x4[hl + 32 * t];
    for (int r0 = gw * RPW; r0 < a.total_rows; r0 += nw * RPW) {
        f32x4 w[RP][NMAT][NV];
        int seg[RP], row[RP];
#pragma unroll
        for (int p = 0; p < RP; p++) {
            const int vr = min(r0 + 2 * p + half, a.total_rows - 1);
            int s = 0;
            if (a.nseg > 1 && vr >= a.seg[1].tile0) s = 1;
            if (a.nseg > 2 && vr >= a.seg[2].tile0) s = 2;
            seg[p] = s;
            row[p] = vr - a.seg[s].tile0;
#pragma unroll
            for (int m = 0; m < NMAT; m++) {
                const f32x4* wr = (const f32x4*)(m == 0 ? a.seg[s].w : a.seg[s].w2) + (int64_t)row[p] * n4;
#pragma unroll
                for (int t = 0; t < NV; t++) w[p][m][t] = gld_nt(wr + hl + 32 * t);
            }
        }
#pragma unroll
        for (int p = 0; p < RP; p++) {
            float v[2];
#pragma unroll
            for (int m = 0; m < NMAT; m++) {
                float s0 = 0.f, s1 = 0.f;
#pragma unroll
                for (int t = 0; t < NV; t++) {
                    float& acc = (t & 1) ? s1 : s0;
                    acc = fmaf(xv[t].x, w[p][m][t].x, acc); acc = fmaf(xv[t].y, w[p][m][t].y, acc);
                    acc = fmaf(xv[t].z, w[p][m][t].z, acc); acc = fmaf(xv[t].w, w[p][m][t].w, acc);
                }
                float h = sum16(s0 + s1);
                h += dpp_rows<0x142, 0xA>(h);   // row_bcast:15: lane 31 = lanes 0..31, lane 63 = 32..63
                v[m] = h;
            }
            if (hl == 31 && r0 + 2 * p + half < a.total_rows) {
                float* y = a.seg[seg[p]].y + row[p];
                if (NMAT == 2) gst(y, silu_mul(v[0], v[1]));
                else if (a.epi == RINA_EPI_ADD) gst(y, gld(y) + v[0]);
                else gst(y, v[0]);
                best = umax64(best, argmax_cand(v[0], row[p]));
            }
        }
    }
}

// NV > 0: rows of K <= 2048 (f32_rows_short); HALF: the half-wave rows
// K > 2048 or unaligned rows: one row per wave per step
template <int NMAT, bool VEC>
__device__ __forceinline__ void f32_rows_loop(const F32Args& a, const float* xs_lds, int gw, int nw,
                                              unsigned long long& best) {
    const int lane = threadIdx.x & 63;
    const int K = a.K;
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
            if (NMAT == 2) gst(y, silu_mul(v[0], v[1]));
            else if (a.epi == RINA_EPI_ADD) gst(y, gld(y) + v[0]);
            else gst(y, v[0]);
            best = umax64(best, argmax_cand(v[0], row));
        }
    }
}

// AM: also the greedy argmax's per-workgroup keys (one segment, store
// epilogue): every workgroup writes the largest key of the rows it stored
// to a.keys[blockIdx.x] (0 when it had none), which argmax_embed_kernel
// reduces.  Only lanes that store a row form keys; the other lanes' keys
// stay 0.
template <int NMAT, bool VEC, int NV, bool HALF = false, bool AM = false>
__global__ __launch_bounds__(kWG) void gemv_f32_kernel(F32Args a) {
    extern __shared__ __align__(16) float xs_lds[];
    __shared__ float red[8];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int K = a.K;
    stage_lds(xs_lds, a.x, K);
    if (a.pro != RINA_PRO_NONE) {   // RMSNorm / LayerNorm of x, in LDS
        __syncthreads();
        float mean = 0.f;
        if (a.pro == RINA_PRO_LAYERNORM) {
            float sm = 0.f;
            for (int i = tid; i < K; i += kWG) sm += xs_lds[i];
            sm = wave_sum(sm);
            if (lane == 0) red[wave] = sm;
            __syncthreads();
            mean = (red[0] + red[1] + red[2] + red[3]) / (float)K;
            __syncthreads();
        }
        float ss = 0.f;
        for (int i = tid; i < K; i += kWG) {
            float t = xs_lds[i] - mean;
            ss = fmaf(t, t, ss);
        }
        ss = wave_sum(ss);
        if (lane == 0) red[4 + wave] = ss;
        __syncthreads();
        float inv = 1.0f / sqrtf((red[4] + red[5] + red[6] + red[7]) / (float)K + a.eps);
        for (int i = tid; i < K; i += kWG) xs_lds[i] = (xs_lds[i] - mean) * inv * gld(a.nw + i);
    }
    __syncthreads();
    const int gw = blockIdx.x * 4 + wave, nw = gridDim.x * 4;
    unsigned long long best = 0ull;
    if constexpr (HALF) {
        f32_rows_half<NMAT, NV, NMAT == 2 ? 2 : 4>(a, xs_lds, gw, nw, best);
    } else if constexpr (NV > 0) {
        f32_rows_short<NMAT, NV>(a, xs_lds, gw, nw, best);
    } else {
        f32_rows_loop<NMAT, VEC>(a, xs_lds, gw, nw, best);
    }
    if constexpr (AM) {
        __shared__ unsigned long long kred[4];
        for (int off = 32; off > 0; off >>= 1) best = umax64(best, __shfl_xor(best, off));
        if (lane == 0) kred[wave] = best;
        __syncthreads();
        if (tid == 0) gst(a.keys + blockIdx.x, umax64(umax64(kred[0], kred[1]), umax64(kred[2], kred[3])));
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
// M >= 16 with Q4 weights on the matrix cores (prompt phase):
// v_mfma_f32_16x16x4f32 over BM x 64 output tiles (BM 64, or 32 when 64-row
// tiles would leave fewer than two workgroups per CU), K stepped by one
// 32-value block.  The x tile and the dequantized weight tile ((q - 7) * scale, the
// reference dequant's per-element value) sit in LDS as fp32, K-major with a
// row stride of 80 floats (a 64-lane fragment read touches every bank
// twice), so each product is the reference's fp32 product and the matrix
// cores accumulate in fp32 (the sums in another order).  Wave w owns the
// (BM / 2) x 32 quarter (w / 2, w % 2) as (BM / 32) x 2 MFMA tiles per
// matrix; the next
// block's x values and weight bytes are loaded into registers while the
// current block is multiplied.
// MFMA operand layout (16x16x4 f32): lane l supplies A[l % 16][l / 16] and
// B[l / 16][l % 16]; result element e of lane l is D[4 (l / 16) + e][l % 16].
// ---------------------------------------------------------------------------
typedef float f32x4m __attribute__((ext_vector_type(4)));

constexpr int kMfmaLd = 80;

// Up to 3 weight segments sharing x (q / k / v) in one launch: column
// tiles t0[s] .. of segment s, in order.
// XCD-aware tile order: workgroups go to the 8 XCDs round-robin in linear
// order, so workgroup id serves XCD id % 8.  The x rows are split into xa
// parts and the weight columns into xb parts (xa * xb = 8); XCD x takes
// m-tiles of part x / xb and n-tiles of part x % xb, so each L2 fetches
// 1/xa of the activation tiles and 1/xb of the weight tiles (the host
// picks the split with the fewest bytes fetched).
struct MfmaArgs {
    GemmArgs g;                  // g.w / g.w2 / g.y / g.N: segment 0
    const uint8_t* w[3];
    float* y[3];
    int N[3];
    int t0[3];
    int nseg;
    int mt, nt;                  // m-tiles, n-tiles
    int xb;                      // weight parts (8 / xb activation parts)
    int mpp, npp;                // m-tiles, n-tiles per part
};

template <int FMT, int NMAT, int BM>
__global__ __launch_bounds__(256) void gemm_mfma_kernel(MfmaArgs ma) {
    constexpr int BB = FMT == FMT_Q4_0F ? 20 : 18;
    constexpr int MI = BM / 32;                    // MFMA tiles per wave along M
    __shared__ float xs[32][kMfmaLd];
    __shared__ float ws[NMAT][32][kMfmaLd];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // this workgroup's tile: XCD id % 8 owns activation part (id % 8) / xb
    // and weight part (id % 8) % xb
    const int xcd = blockIdx.x & 7, k = blockIdx.x >> 3;
    const int mm = k / ma.npp, nn = k - mm * ma.npp;
    const int by = (xcd / ma.xb) * ma.mpp + mm, bx = (xcd % ma.xb) * ma.npp + nn;
    if (mm >= ma.mpp || by >= ma.mt || bx >= ma.nt) return;   // padding of the split
    // this workgroup's segment (wave-uniform selects, no indexed argument reads)
    GemmArgs a = ma.g;
    const int sg = (ma.nseg > 1 && bx >= ma.t0[1]) + (ma.nseg > 2 && bx >= ma.t0[2]);
    a.w = sg == 0 ? ma.w[0] : sg == 1 ? ma.w[1] : ma.w[2];
    a.y = sg == 0 ? ma.y[0] : sg == 1 ? ma.y[1] : ma.y[2];
    a.N = sg == 0 ? ma.N[0] : sg == 1 ? ma.N[1] : ma.N[2];
    const int tb = sg == 0 ? ma.t0[0] : sg == 1 ? ma.t0[1] : ma.t0[2];
    const int m0 = by * BM, n0 = (bx - tb) * 64;
    const int nb = a.K / 32;
    // staging: thread t takes row t / 4 of the x tile (rows < BM) and of
    // each weight tile, values 8 (t % 4) .. 8 (t % 4) + 7 of the block
    const int sr = tid >> 2, sq = tid & 3;
    const bool xok = sr < BM && m0 + sr < a.M, wok = n0 + sr < a.N;
    const float* xrow = a.x + (int64_t)(xok ? m0 + sr : 0) * a.K + 8 * sq;
    const int64_t wrow = (int64_t)(wok ? n0 + sr : 0) * nb * BB;
    // Q2_K (flat element order): values 8 sq .. 8 sq + 7 of the row's block b
    // are elements e = row K + 32 b + 8 sq, inside one 256-value block and
    // one shift group g of one 128-value page (row starts and b are
    // multiples of 32): qs bytes 16 + 32 page + 8 sq .. + 7, scale byte
    // 8 page + sq / 2 + 2 g, fp16 d / dmin at 80 / 82
    const int64_t erow = (int64_t)(wok ? n0 + sr : 0) * a.K + 8 * sq;
    f32x4 xr0, xr1;
    uint32_t wsc[NMAT], wnb[NMAT], wq1[NMAT], wdd[NMAT];
    auto load_blk = [&](int b) {
        const f32x4* xp = (const f32x4*)(xrow + 32 * b);
        xr0 = gld(xp);
        xr1 = gld(xp + 1);
#pragma unroll
        for (int m = 0; m < NMAT; m++) {
            if constexpr (FMT == FMT_Q2_K) {
                const int64_t e = erow + 32 * b;
                const uint8_t* bd = (m ? a.w2 : a.w) + (e >> 8) * 84;
                const int inb = (int)(e & 255), page = inb >> 7, g = (inb & 127) >> 5;
                const int is = 8 * page + (sq >> 1) + 2 * g;
                wnb[m] = gld((const uint32_t*)(bd + 16 + 32 * page + 8 * sq));
                wq1[m] = gld((const uint32_t*)(bd + 20 + 32 * page + 8 * sq));
                wsc[m] = ((gld((const uint32_t*)(bd + (is & ~3))) >> (8 * (is & 3))) & 0xFF) | ((uint32_t)(2 * g) << 8);
                wdd[m] = gld((const uint32_t*)(bd + 80));
            } else {
                const uint8_t* bp = (m ? a.w2 : a.w) + wrow + (int64_t)b * BB;
                if constexpr (FMT == FMT_Q4_0F) {
                    wsc[m] = gld((const uint32_t*)bp);
                    wnb[m] = gld((const uint32_t*)(bp + 4 + 4 * sq));
                } else {
                    wsc[m] = gld((const uint16_t*)bp);
                    wnb[m] = (uint32_t)gld((const uint16_t*)(bp + 2 + 4 * sq)) |
                             ((uint32_t)gld((const uint16_t*)(bp + 4 + 4 * sq)) << 16);
                }
            }
        }
    };
    // value 8 sq + t of the block is nibble t of wnb (byte t / 2, low nibble for even t)
    auto store_blk = [&]() {
        const float xv[8] = {xr0.x, xr0.y, xr0.z, xr0.w, xr1.x, xr1.y, xr1.z, xr1.w};
        if (sr < BM) {
#pragma unroll
            for (int t = 0; t < 8; t++) xs[8 * sq + t][sr] = xok ? xv[t] : 0.f;
        }
#pragma unroll
        for (int m = 0; m < NMAT; m++) {
            if constexpr (FMT == FMT_Q2_K) {
                // ops/linear.cu:413-431: d * (sc & 15) * q - dmin * (sc >> 4)
                const uint32_t sc = wsc[m] & 0xFF, sh = wsc[m] >> 8;
                const float dv = f16_to_f32((uint16_t)(wdd[m] & 0xFFFF)), mv = f16_to_f32((uint16_t)(wdd[m] >> 16));
                const float scale = dv * (float)(sc & 0xF), mn = mv * (float)(sc >> 4);
#pragma unroll
                for (int t = 0; t < 8; t++) {
                    const uint32_t qb = ((t < 4 ? wnb[m] : wq1[m]) >> (8 * (t & 3))) & 0xFF;
                    ws[m][8 * sq + t][sr] = wok ? fmaf(scale, (float)((qb >> sh) & 3), -mn) : 0.f;
                }
            } else {
                const float sc = FMT == FMT_Q4_0F ? __uint_as_float(wsc[m]) : f16_to_f32((uint16_t)wsc[m]);
#pragma unroll
                for (int t = 0; t < 8; t++)
                    ws[m][8 * sq + t][sr] = wok ? (float)((int)((wnb[m] >> (4 * t)) & 0xF) - 7) * sc : 0.f;
            }
        }
    };
    const int wm = (wave >> 1) * 16 * MI, wn = (wave & 1) * 32;
    const int fr = lane & 15, fk = lane >> 4;
    f32x4m acc[NMAT][MI][2];
#pragma unroll
    for (int m = 0; m < NMAT; m++)
#pragma unroll
        for (int i = 0; i < MI; i++)
#pragma unroll
            for (int j = 0; j < 2; j++) acc[m][i][j] = f32x4m{0.f, 0.f, 0.f, 0.f};
    load_blk(0);
    for (int b = 0; b < nb; b++) {
        __syncthreads();                           // the previous block's fragments are read
        store_blk();
        __syncthreads();
        load_blk(b + 1 < nb ? b + 1 : b);          // unconditional: the last block reloads itself
#pragma unroll
        for (int kk = 0; kk < 8; kk++) {
            const int k = 4 * kk + fk;
            float av[MI];
#pragma unroll
            for (int i = 0; i < MI; i++) av[i] = xs[k][wm + 16 * i + fr];
#pragma unroll
            for (int m = 0; m < NMAT; m++) {
                const float b0 = ws[m][k][wn + fr], b1 = ws[m][k][wn + 16 + fr];
#pragma unroll
                for (int i = 0; i < MI; i++) {
                    acc[m][i][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i], b0, acc[m][i][0], 0, 0, 0);
                    acc[m][i][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i], b1, acc[m][i][1], 0, 0, 0);
                }
            }
        }
    }
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int row = m0 + wm + 16 * i + 4 * fk + e, col = n0 + wn + 16 * j + fr;
                if (row >= a.M || col >= a.N) continue;
                float* y = a.y + (int64_t)row * a.N + col;
                const float v0 = acc[0][i][j][e];
                if (NMAT == 2) *y = silu_mul(v0, acc[NMAT - 1][i][j][e]);
                else if (a.epi == RINA_EPI_ADD) *y = *y + v0;
                else *y = v0;
            }
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// the high halves of two fp32 bit patterns as one dword of two bf16 (a's in
// the low half)
__device__ __forceinline__ uint32_t hi16_pair(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x07060302u); }

// x0, x1 split into three bf16 parts each, x = h + m + l: h is x cut to its
// top 8 significant bits, m the remainder cut the same way, l the rest (at
// most 8 significant bits); packed as two-value dwords.  Exact for finite
// |x| >= 2^-103 and for 0, where both remainders are normal fp32 values; an
// infinite x gives NaN parts (inf - inf), and a smaller x loses low bits of
// l (the matrix cores may also flush bf16 denormals)
__device__ __forceinline__ void split3_pair(float x0, float x1, uint32_t& ph, uint32_t& pm, uint32_t& pl) {
    const uint32_t u0 = __float_as_uint(x0), u1 = __float_as_uint(x1);
    ph = hi16_pair(u0, u1);
    const float r0 = x0 - __uint_as_float(u0 & 0xFFFF0000u), r1 = x1 - __uint_as_float(u1 & 0xFFFF0000u);
    const uint32_t v0 = __float_as_uint(r0), v1 = __float_as_uint(r1);
    pm = hi16_pair(v0, v1);
    const float s0 = r0 - __uint_as_float(v0 & 0xFFFF0000u), s1 = r1 - __uint_as_float(v1 & 0xFFFF0000u);
    pl = hi16_pair(__float_as_uint(s0), __float_as_uint(s1));
}

// Prompt matmul for Q4_0 / Q4_0F weights on the bf16 matrix cores, with fp32
// products and sums.  Every x value is split exactly into three bf16 parts,
// x = h + m + l (8 significant bits each: the two remainders are exact in
// fp32), and a weight value q - 7 is a small integer, exact in bf16, so
// v_mfma_f32_16x16x32_bf16 forms the exact products of the fp32 x with the
// integer weights and sums them in fp32.  Per 32-value block and 16x16 tile
// three MFMAs (l, m, h into one accumulator), then one fp32 fma with the
// block scale of the tile column.  XCD order, segments and epilogues as
// gemm_mfma_kernel; tiles are BM x 32 WN with 2 WN waves (two down the rows,
// WN across, each wave 16 MI rows x 32 columns), so one split of an x tile
// serves 32 WN columns.  LDS rows of (32 * KB + 8) bf16 keep the 16-byte
// fragment reads of 16 rows on distinct banks.  Fragment layout (16x16x32): lane l holds
// A[l % 16][8 (l / 16) .. + 7], B[8 (l / 16) .. + 7][l % 16] and
// D[4 (l / 16) + e][l % 16].
template <int FMT, int NMAT, int BM, int WN>
__global__ __launch_bounds__(128 * WN) void gemm_bf3_kernel(MfmaArgs ma) {
    constexpr int BB = FMT == FMT_Q4_0F ? 20 : 18;
    constexpr int MI = BM / 32;                    // MFMA tiles per wave along M
    // 32-value blocks per LDS stage: four cut the barriers of the one-matrix
    // launches (two at 64 rows, whose LDS would otherwise hold one
    // workgroup per CU); the paired SwiGLU tile keeps one (its registers
    // would cut occupancy to 3 waves per SIMD)
    constexpr int KB = NMAT == 2 ? 1 : BM == 64 ? 2 : 4;
    constexpr int LD = 32 * KB + 8;
    // WN waves across the tile's columns (32 each) and two down its rows
    constexpr int BN = 32 * WN, NT = 128 * WN;
    __shared__ __align__(16) uint16_t xs[3][BM][LD];
    __shared__ __align__(16) uint16_t ws[NMAT][BN][LD];
    __shared__ float wsc_s[NMAT][KB][BN];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int xcd = blockIdx.x & 7, k = blockIdx.x >> 3;
    const int mm = k / ma.npp, nn = k - mm * ma.npp;
    const int by = (xcd / ma.xb) * ma.mpp + mm, bx = (xcd % ma.xb) * ma.npp + nn;
    if (mm >= ma.mpp || by >= ma.mt || bx >= ma.nt) return;   // padding of the split
    GemmArgs a = ma.g;
    const int sg = (ma.nseg > 1 && bx >= ma.t0[1]) + (ma.nseg > 2 && bx >= ma.t0[2]);
    a.w = sg == 0 ? ma.w[0] : sg == 1 ? ma.w[1] : ma.w[2];
    a.y = sg == 0 ? ma.y[0] : sg == 1 ? ma.y[1] : ma.y[2];
    a.N = sg == 0 ? ma.N[0] : sg == 1 ? ma.N[1] : ma.N[2];
    const int tb = sg == 0 ? ma.t0[0] : sg == 1 ? ma.t0[1] : ma.t0[2];
    const int m0 = by * BM, n0 = (bx - tb) * BN;
    const int nb = a.K / 32, nst = (nb + KB - 1) / KB;
    // x staging: every thread splits XV values of one row per block (XT
    // threads per row), so the split work is spread over all the waves;
    // weight staging: thread tid takes values 8 sq .. 8 sq + 7 of column sr
    constexpr int XV = BM * 32 / NT, XT = 32 / XV;
    const int xsr = tid / XT, xsq = tid % XT;
    const int sr = tid >> 2, sq = tid & 3;
    const bool xok = m0 + xsr < a.M, wok = n0 + sr < a.N;
    const float* xrow = a.x + (int64_t)(xok ? m0 + xsr : 0) * a.K + XV * xsq;
    const int64_t wrow = (int64_t)(wok ? n0 + sr : 0) * nb * BB;
    // register sets holding one stage's loads each; with two, a stage's loads
    // are issued two stages before they are stored to LDS
    struct Stage {
        float xr[KB][XV];
        uint32_t wsc[KB][NMAT], wnb[KB][NMAT];
    };
    Stage r0, r1;
    // stage st: blocks KB st .. KB st + KB - 1 (past nb: block nb - 1 again,
    // stored as zeros)
    auto load_stage = [&](Stage& r, int st) {
#pragma unroll
        for (int kb = 0; kb < KB; kb++) {
            const int b = min(KB * st + kb, nb - 1);
            if constexpr (XV >= 4) {
                const f32x4* xp = (const f32x4*)(xrow + 32 * b);
#pragma unroll
                for (int v = 0; v < XV / 4; v++) {
                    const f32x4 t = gld(xp + v);
                    r.xr[kb][4 * v] = t.x; r.xr[kb][4 * v + 1] = t.y; r.xr[kb][4 * v + 2] = t.z; r.xr[kb][4 * v + 3] = t.w;
                }
            } else {
                const f32x2 t = gld((const f32x2*)(xrow + 32 * b));
                r.xr[kb][0] = t.x; r.xr[kb][1] = t.y;
            }
#pragma unroll
            for (int m = 0; m < NMAT; m++) {
                const uint8_t* bp = (m ? a.w2 : a.w) + wrow + (int64_t)b * BB;
                if constexpr (FMT == FMT_Q4_0F) {
                    r.wsc[kb][m] = gld((const uint32_t*)bp);
                    r.wnb[kb][m] = gld((const uint32_t*)(bp + 4 + 4 * sq));
                } else {
                    r.wsc[kb][m] = gld((const uint16_t*)bp);
                    r.wnb[kb][m] = (uint32_t)gld((const uint16_t*)(bp + 2 + 4 * sq)) |
                                 ((uint32_t)gld((const uint16_t*)(bp + 4 + 4 * sq)) << 16);
                }
            }
        }
    };
    // value 8 sq + t of a block is nibble t of wnb (byte t / 2, low nibble for even t)
    auto store_stage = [&](const Stage& r, int st) {
#pragma unroll
        for (int kb = 0; kb < KB; kb++) {
            const bool bok = KB * st + kb < nb;
            {
                float xv[XV];
#pragma unroll
                for (int v = 0; v < XV; v++) xv[v] = r.xr[kb][v];
                const bool on = xok && bok;
                uint32_t ph[XV / 2], pm[XV / 2], pl[XV / 2];
#pragma unroll
                for (int t = 0; t < XV; t += 2)
                    split3_pair(on ? xv[t] : 0.f, on ? xv[t + 1] : 0.f, ph[t >> 1], pm[t >> 1], pl[t >> 1]);
                uint16_t* d0 = &xs[0][xsr][32 * kb + XV * xsq];
                uint16_t* d1 = &xs[1][xsr][32 * kb + XV * xsq];
                uint16_t* d2 = &xs[2][xsr][32 * kb + XV * xsq];
                if constexpr (XV == 8) {
                    *(u32x4*)d0 = u32x4{ph[0], ph[1], ph[2], ph[3]};
                    *(u32x4*)d1 = u32x4{pm[0], pm[1], pm[2], pm[3]};
                    *(u32x4*)d2 = u32x4{pl[0], pl[1], pl[2], pl[3]};
                } else if constexpr (XV == 2) {
                    *(uint32_t*)d0 = ph[0];
                    *(uint32_t*)d1 = pm[0];
                    *(uint32_t*)d2 = pl[0];
                } else {
                    *(u32x2*)d0 = u32x2{ph[0], ph[1]};
                    *(u32x2*)d1 = u32x2{pm[0], pm[1]};
                    *(u32x2*)d2 = u32x2{pl[0], pl[1]};
                }
            }
#pragma unroll
            for (int m = 0; m < NMAT; m++) {
                // q - 7 as bf16, a small integer (exact): nibble t of wnb is
                // byte t / 2 of lo (even t) or hi (odd t)
                const uint32_t lo = and_opaque(r.wnb[kb][m], 0x0F0F0F0Fu), hi = and_opaque(r.wnb[kb][m] >> 4, 0x0F0F0F0Fu);
                uint32_t pw[4];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const float f0 = (float)((lo >> (8 * j)) & 0xFF) - 7.0f, f1 = (float)((hi >> (8 * j)) & 0xFF) - 7.0f;
                    pw[j] = wok && bok ? hi16_pair(__float_as_uint(f0), __float_as_uint(f1)) : 0u;
                }
                *(u32x4*)&ws[m][sr][32 * kb + 8 * sq] = u32x4{pw[0], pw[1], pw[2], pw[3]};
                if (sq == 0) {
                    const float sc = FMT == FMT_Q4_0F ? __uint_as_float(r.wsc[kb][m]) : f16_to_f32((uint16_t)r.wsc[kb][m]);
                    wsc_s[m][kb][sr] = wok && bok ? sc : 0.f;
                }
            }
        }
    };
    const int wm = (wave / WN) * 16 * MI, wn = (wave % WN) * 32;
    const int fr = lane & 15, fk = lane >> 4;
    f32x4m acc[NMAT][MI][2];
#pragma unroll
    for (int m = 0; m < NMAT; m++)
#pragma unroll
        for (int i = 0; i < MI; i++)
#pragma unroll
            for (int j = 0; j < 2; j++) acc[m][i][j] = f32x4m{0.f, 0.f, 0.f, 0.f};
    auto compute_stage = [&]() {
#pragma unroll
        for (int kb = 0; kb < KB; kb++) {
            bf16x8 af[3][MI];
#pragma unroll
            for (int p = 0; p < 3; p++)
#pragma unroll
                for (int i = 0; i < MI; i++) af[p][i] = *(const bf16x8*)&xs[p][wm + 16 * i + fr][32 * kb + 8 * fk];
#pragma unroll
            for (int m = 0; m < NMAT; m++)
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const bf16x8 bf = *(const bf16x8*)&ws[m][wn + 16 * j + fr][32 * kb + 8 * fk];
                    const float sc = wsc_s[m][kb][wn + 16 * j + fr];
#pragma unroll
                    for (int i = 0; i < MI; i++) {
                        f32x4m d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[2][i], bf, f32x4m{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[1][i], bf, d, 0, 0, 0);
                        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[0][i], bf, d, 0, 0, 0);
#pragma unroll
                        for (int e = 0; e < 4; e++) acc[m][i][j][e] = fmaf(sc, d[e], acc[m][i][j][e]);
                    }
                }
        }
    };
    load_stage(r0, 0);
    if constexpr (NMAT == 1) {
        // stages in pairs, unconditionally: with nst odd the last pair's
        // second stage lies past nb, is stored as zeros and adds sc 0 times d 0
        load_stage(r1, 1);
        for (int st = 0; st < nst; st += 2) {
            __syncthreads();                       // the previous stage's fragments are read
            store_stage(r0, st);
            __syncthreads();
            load_stage(r0, st + 2);
            compute_stage();
            __syncthreads();
            store_stage(r1, st + 1);
            __syncthreads();
            load_stage(r1, st + 3);
            compute_stage();
        }
    } else {
        // the paired SwiGLU tile keeps one register set (a second would cut
        // occupancy from 5 to 3 waves per SIMD, which costs it more)
        for (int st = 0; st < nst; st++) {
            __syncthreads();
            store_stage(r0, st);
            __syncthreads();
            load_stage(r0, st + 1);                // past the end: block nb - 1, not stored
            compute_stage();
        }
    }
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int row = m0 + wm + 16 * i + 4 * fk + e, col = n0 + wn + 16 * j + fr;
                if (row >= a.M || col >= a.N) continue;
                float* y = a.y + (int64_t)row * a.N + col;
                const float v0 = acc[0][i][j][e];
                if (NMAT == 2) *y = silu_mul(v0, acc[NMAT - 1][i][j][e]);
                else if (a.epi == RINA_EPI_ADD) *y = *y + v0;
                else *y = v0;
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

template <int FMT, int WPR, int CPL, int NMAT, int PRO>
int launch_quant(GemvArgs& a, hipStream_t st) {
    int cus = rina_num_cus();
    int grid = a.total_tiles < cus * 4 ? a.total_tiles : cus * 4;
    size_t lds = 2 * (size_t)NMAT * a.slot + (size_t)NMAT * a.R * WPR * 4;
    hipLaunchKernelGGL((gemv_quant_kernel<FMT, WPR, CPL, NMAT, PRO>), dim3(grid), dim3(kWG), lds, st, a);
    return hipGetLastError() == hipSuccess ? RINA_OK : RINA_ERR_HIP;
}

template <int FMT, int NMAT>
int dispatch_wpr(GemvArgs& a, int wpr, int cpl, int pro, hipStream_t st) {
    if (wpr == 1 && cpl == 1) {
        if (pro == RINA_PRO_RMSNORM) return launch_quant<FMT, 1, 1, NMAT, RINA_PRO_RMSNORM>(a, st);
        if (pro == RINA_PRO_LAYERNORM) return launch_quant<FMT, 1, 1, NMAT, RINA_PRO_LAYERNORM>(a, st);
        return launch_quant<FMT, 1, 1, NMAT, 0>(a, st);
    }
    if (pro != RINA_PRO_NONE) return RINA_ERR_SHAPE;
    if (wpr == 2) return cpl == 1 ? launch_quant<FMT, 2, 1, NMAT, 0>(a, st) : RINA_ERR_SHAPE;
    switch (cpl) {
        case 1: return launch_quant<FMT, 4, 1, NMAT, 0>(a, st);
        case 2: return launch_quant<FMT, 4, 2, NMAT, 0>(a, st);
        case 3: return launch_quant<FMT, 4, 3, NMAT, 0>(a, st);
        case 4: return launch_quant<FMT, 4, 4, NMAT, 0>(a, st);
        default: return RINA_ERR_SHAPE;
    }
}

template <int FMT, int WPR, int NMAT, int PRO, int RB, int NS>
int launch_direct(GemvArgs& a, hipStream_t st) {
    constexpr int RPI = 4 / WPR;
    int cus = rina_num_cus();
    int wgs = (a.total_tiles + RPI - 1) / RPI;
    // workgroups per CU (measured): Q2_K with 4 rows and one matrix (89
    // VGPRs, 28.7 KB of LDS) takes 5, the LM head 102400 x 2048 measured
    // 32.5 / 31.5 / 30.8 us at 3 / 4 / 5; Q4 with 1-4 rows per wave takes 3
    // (config 1 8192 x 2048 at 2 rows: 4.42 us at 4, 4.28 at 3; SwiGLU
    // 8192 x 2048 at 1 row: 7.33 / 6.44 us), 8 rows take 2
    int per_cu = FMT == FMT_Q2_K ? (RB >= 4 ? (NMAT == 2 ? 2 : 5) : 4) : (RB >= 8 ? 2 : 3);
    int grid = wgs < cus * per_cu ? wgs : cus * per_cu;
    // one iteration per workgroup: straight-line code; more: the two-set loop.
    // Measured on the config-2 shapes: every iteration's loads issued at
    // entry (2-3 iterations) made the launches slower (SwiGLU 8192 x 2048
    // 6.5 -> 7.9 us, config 1 4.4 -> 5.1 us), also with a barrier that puts
    // every wave's activation requests ahead of the weight requests
    // (SwiGLU 7.85 us), and so did two groups in flight from entry in the
    // two-set loop (SwiGLU 7.0 us, config 1 5.1 us): the activation loads of
    // a CU's later waves then queue behind more weight requests.
    const bool one = wgs <= grid;
    // residual epilogue: the old output words are loaded with the weights
    // (W_o 3.16 -> 2.99 us, W2 5.5 -> 5.2 us); a store epilogue loads none
    // (the same loads cost the fused q/k/v 3.35 -> 3.75 us)
    const bool yl = NMAT == 1 && a.epi == RINA_EPI_ADD;
    if (one) {
        if (yl) hipLaunchKernelGGL((gemv_direct_kernel<FMT, WPR, NMAT, PRO, RB, NS, 1, true>), dim3(grid), dim3(kWG), 0, st, a);
        else hipLaunchKernelGGL((gemv_direct_kernel<FMT, WPR, NMAT, PRO, RB, NS, 1, false>), dim3(grid), dim3(kWG), 0, st, a);
    } else {
        if (yl) hipLaunchKernelGGL((gemv_direct_kernel<FMT, WPR, NMAT, PRO, RB, NS, 0, true>), dim3(grid), dim3(kWG), 0, st, a);
        else hipLaunchKernelGGL((gemv_direct_kernel<FMT, WPR, NMAT, PRO, RB, NS, 0, false>), dim3(grid), dim3(kWG), 0, st, a);
    }
    return hipGetLastError() == hipSuccess ? RINA_OK : RINA_ERR_HIP;
}

template <int FMT, int WPR, int NMAT, int PRO>
int direct_rb(GemvArgs& a, int rb, hipStream_t st) {
    if (a.nseg > 3) {   // more than 3 segments: the 6-segment table, 1 or 2 rows per wave
        if constexpr (NMAT == 1) {
            return rb <= 1 ? launch_direct<FMT, WPR, 1, PRO, 1, kMaxDirectSegs>(a, st)
                           : launch_direct<FMT, WPR, 1, PRO, 2, kMaxDirectSegs>(a, st);
        }
        return RINA_ERR_ARG;
    }
    // one matrix in one segment: no per-row segment selection (graph
    // replays over weight rings past the MALL: W_o 2048 x 2048 3.05 -> 2.92
    // us, W2 2048 x 8192 5.50 -> 5.25, the Q2_K LM head 102400 x 2048 31.5
    // -> 29.2, whose 3-segment form spilled scalar registers; the SwiGLU
    // pair 8192 x 2048 measured slower in this form, 6.80 -> 7.03)
    if constexpr (NMAT == 1) {
        if (a.nseg == 1) {
            switch (rb) {
                case 1: return launch_direct<FMT, WPR, 1, PRO, 1, 1>(a, st);
                case 2: return launch_direct<FMT, WPR, 1, PRO, 2, 1>(a, st);
                case 4: return launch_direct<FMT, WPR, 1, PRO, 4, 1>(a, st);
                default: return launch_direct<FMT, WPR, 1, PRO, (FMT == FMT_Q2_K ? 4 : 8), 1>(a, st);
            }
        }
    }
    switch (rb) {
        case 1: return launch_direct<FMT, WPR, NMAT, PRO, 1, 3>(a, st);
        case 2: return launch_direct<FMT, WPR, NMAT, PRO, 2, 3>(a, st);
        case 4: return launch_direct<FMT, WPR, NMAT, PRO, 4, 3>(a, st);
        default: return launch_direct<FMT, WPR, NMAT, PRO, (FMT == FMT_Q2_K ? 4 : 8), 3>(a, st);
    }
}

template <int FMT, int WPR, int NMAT>
int direct_pro(GemvArgs& a, int rb, int pro, hipStream_t st) {
    if (pro == RINA_PRO_RMSNORM) return direct_rb<FMT, WPR, NMAT, RINA_PRO_RMSNORM>(a, rb, st);
    if (pro == RINA_PRO_LAYERNORM) return direct_rb<FMT, WPR, NMAT, RINA_PRO_LAYERNORM>(a, rb, st);
    return direct_rb<FMT, WPR, NMAT, 0>(a, rb, st);
}

template <int FMT, int NMAT>
int dispatch_direct(GemvArgs& a, int wpr, int rb, int pro, hipStream_t st) {
    if (wpr == 1) return direct_pro<FMT, 1, NMAT>(a, rb, pro, st);
    if (wpr == 2) return direct_pro<FMT, 2, NMAT>(a, rb, pro, st);
    return direct_pro<FMT, 4, NMAT>(a, rb, pro, st);
}

// M = 1 shapes the direct-load kernel takes: 32-value columns, at most one
// per lane of four waves.
// Q2_K: K % 128 == 0 keeps the four lanes of a quad on one half page (the
// quad form of the column loads, 4+ rows per wave)
bool direct_ok(int fmt, int K) { return fmt >= 0 && K % (fmt == FMT_Q2_K ? 128 : 32) == 0 && K <= 8192; }

// waves per row / units per lane for a row of `nunits` work units
void split_row(int nunits, int& wpr, int& cpl) {
    if (nunits <= 64) { wpr = 1; cpl = 1; }
    else if (nunits <= 128) { wpr = 2; cpl = 1; }
    else { wpr = 4; cpl = (nunits + 255) / 256; }
}

int gemv_quant(const rina_linear_seg* segs, int nseg, int qt, const float* x, int K, int epi, int pro,
               const float* nw, float eps, float* xn, hipStream_t st) {
    int fmt = fmt_of(qt);
    int nmat = (epi == RINA_EPI_SWIGLU) ? 2 : 1;
    int unit = fmt == FMT_Q2_K ? 16 : 32;
    if (K % unit) return RINA_ERR_SHAPE;
    int wpr, cpl;
    split_row(K / unit, wpr, cpl);
    if (cpl > 4) return RINA_ERR_SHAPE;
    GemvArgs a{};
    a.nseg = nseg;
    a.x = x;
    a.K = K;
    a.epi = epi;
    a.nw = nw;
    a.eps = eps;
    int64_t rowbytes = fmt == FMT_Q4_0 ? (int64_t)(K / 32) * 18 : fmt == FMT_Q4_0F ? (int64_t)(K / 32) * 20 : 0;
    a.rowbytes = (int)rowbytes;
    if (direct_ok(fmt, K)) {
        split_row(K / 32, wpr, cpl);
        // direct-load kernel: virtual rows over all segments, RB rows per wave
        int rows = 0;
        for (int s = 0; s < nseg; s++) {
            GemvSeg& g = s < 3 ? a.seg[s] : a.seg_hi[s - 3];
            g.w = (const uint8_t*)segs[s].weight;
            g.w2 = (const uint8_t*)segs[s].weight2;
            g.y = segs[s].out;
            g.N = segs[s].N;
            g.tile0 = rows;
            rows += segs[s].N;
        }
        a.xn = pro != RINA_PRO_NONE ? xn : nullptr;
        // rows per wave: about two workgroups per CU (each preps the
        // activation once), up to 8 rows per wave
        int64_t waves = (int64_t)rina_num_cus() * 8;
        int64_t want = ((int64_t)rows * wpr + waves - 1) / waves;
        if (fmt != FMT_Q2_K) {
            // measured on the Q4 decode shapes: two matrices per row want
            // more waves (SwiGLU 8192 x 2048: 2 rows per wave, 8.1 -> 7.5 us);
            // a long row makes every workgroup's activation prep costly, so
            // fewer, fuller workgroups (K 8192: 8 rows, 6.6 -> 5.9 us); single
            // matrices of 2048+ rows take at least 2 rows per wave (W_o
            // 2048 x 2048: 3.4 -> 3.25 us; a 1536-row SwiGLU loses with 2)
            if (nmat == 2) want = (want + 1) / 2;
            if (wpr >= 4) want *= 2;
            if (nmat == 1 && rows >= 2048 && want < 2) want = 2;
        }
        int rb = want <= 1 ? 1 : want <= 2 ? 2 : want <= 4 ? 4 : 8;
        if (fmt == FMT_Q2_K && rb > 4) rb = 4;   // 8 rows measured slower (LM head 32 -> 35 us)
        // Q4 rows of at most 4096 values: more workgroups with fewer rows
        // each (config 1 8192 x 2048: 4 -> 2 rows per wave, 5.06 -> 4.28 us;
        // SwiGLU 8192 x 2048: 2 -> 1 row, 7.22 -> 6.44 us, 3 workgroups per CU)
        if (fmt != FMT_Q2_K && wpr < 4) {
            const int cap = nmat == 2 ? 1 : 2;
            if (rb > cap) rb = cap;
        }
        a.R = rows;
        a.total_tiles = (rows + rb - 1) / rb;
        if (fmt == FMT_Q2_K)
            return nmat == 2 ? dispatch_direct<FMT_Q2_K, 2>(a, wpr, rb, pro, st) : dispatch_direct<FMT_Q2_K, 1>(a, wpr, rb, pro, st);
        if (fmt == FMT_Q4_0)
            return nmat == 2 ? dispatch_direct<FMT_Q4_0, 2>(a, wpr, rb, pro, st) : dispatch_direct<FMT_Q4_0, 1>(a, wpr, rb, pro, st);
        return nmat == 2 ? dispatch_direct<FMT_Q4_0F, 2>(a, wpr, rb, pro, st) : dispatch_direct<FMT_Q4_0F, 1>(a, wpr, rb, pro, st);
    }
    // LDS bytes of one matrix slot for R rows: the rows' byte range, a
    // 16-byte alignment lead, read slack, and for Q2_K one extra block
    // (a tile's rows may straddle 256-value blocks at both ends).
    auto slot_for = [&](int R) -> int64_t {
        int64_t b = fmt == FMT_Q2_K ? (((int64_t)R * K + 255) / 256 + 1) * 84 : (int64_t)R * rowbytes;
        return (b + 32 + 15) & ~15LL;
    };
    int R = 64;
    while (R > 1 && slot_for(R) * nmat > kTileBytes) R--;
    if (slot_for(R) * nmat > kTileBytes) return RINA_ERR_SHAPE;
    a.R = R;
    a.slot = (int)slot_for(R);
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
        case FMT_Q4_0:
            return nmat == 2 ? dispatch_wpr<FMT_Q4_0, 2>(a, wpr, cpl, pro, st) : dispatch_wpr<FMT_Q4_0, 1>(a, wpr, cpl, pro, st);
        case FMT_Q4_0F:
            return nmat == 2 ? dispatch_wpr<FMT_Q4_0F, 2>(a, wpr, cpl, pro, st) : dispatch_wpr<FMT_Q4_0F, 1>(a, wpr, cpl, pro, st);
        default:
            return nmat == 2 ? dispatch_wpr<FMT_Q2_K, 2>(a, wpr, cpl, pro, st) : dispatch_wpr<FMT_Q2_K, 1>(a, wpr, cpl, pro, st);
    }
}

// keys != NULL: one segment, store epilogue, and the argmax keys of every
// workgroup into keys[0 .. *nkeys) (at most max_keys)
int gemv_f32(const rina_linear_seg* segs, int nseg, const float* x, int K, int epi, int pro, const float* nw,
             float eps, hipStream_t st, unsigned long long* keys = nullptr, int max_keys = 0, int* nkeys = nullptr) {
    F32Args a{};
    a.keys = keys;
    a.pro = pro;
    a.nw = nw;
    a.eps = eps;
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
    // short rows (K <= 2048, 16-byte aligned): several rows per wave with all
    // loads in flight; NV = 16-byte loads per lane per row
    const int nv = vec && K <= 2048 ? (K / 4 + 63) / 64 : 0;
    // K / 4 an odd multiple of 32 (K = 128, 384, 640, 896): half-wave rows
    const int nvh = vec && (K / 4) % 64 == 32 && K <= 896 ? K / 128 : 0;
    if (nvh > 0) {
        const int rpw = two ? 4 : 8;
        int g2 = (rows + 4 * rpw - 1) / (4 * rpw);
        if (g2 < grid) grid = g2;
    } else if (nv > 0) {
        const int rpw = two ? 2 : 4;
        int g2 = (rows + 4 * rpw - 1) / (4 * rpw);
        if (g2 < grid) grid = g2;
        // 4 workgroups per CU (the LM head 128256 x 2048 over copies past
        // the MALL: 155.0-155.9 us against 156.3-159.2 at 8 and 156.5-157.6
        // at 2; the half-wave rows above keep 8: K 640 49.9-50.2 us against
        // 50.5-50.9 at 4)
        if (grid > cus * 4) grid = cus * 4;
    }
    if (keys) {
        if (nseg != 1 || epi != RINA_EPI_STORE) return RINA_ERR_ARG;
        if (grid > max_keys) return RINA_ERR_WORKSPACE;
        *nkeys = grid;
#define F32_AM(V, NVV, H) hipLaunchKernelGGL((gemv_f32_kernel<1, V, NVV, H, true>), dim3(grid), dim3(kWG), lds, st, a)
        if (nvh > 0) {
            switch (nvh) {
                case 1: F32_AM(true, 1, true); break;
                case 3: F32_AM(true, 3, true); break;
                case 5: F32_AM(true, 5, true); break;
                default: F32_AM(true, 7, true); break;
            }
        } else if (nv > 0) {
            switch (nv <= 2 ? 2 : nv <= 4 ? 4 : 8) {
                case 2: F32_AM(true, 2, false); break;
                case 4: F32_AM(true, 4, false); break;
                default: F32_AM(true, 8, false); break;
            }
        } else if (vec) {
            F32_AM(true, 0, false);
        } else {
            F32_AM(false, 0, false);
        }
#undef F32_AM
        return hipGetLastError() == hipSuccess ? RINA_OK : RINA_ERR_HIP;
    }
#define F32_LAUNCH(NM, V, NVV) hipLaunchKernelGGL((gemv_f32_kernel<NM, V, NVV>), dim3(grid), dim3(kWG), lds, st, a)
#define F32_HALF(NM, NVV) hipLaunchKernelGGL((gemv_f32_kernel<NM, true, NVV, true>), dim3(grid), dim3(kWG), lds, st, a)
    if (nvh > 0) {
        switch (nvh * (two ? -1 : 1)) {
            case 1: F32_HALF(1, 1); break;
            case 3: F32_HALF(1, 3); break;
            case 5: F32_HALF(1, 5); break;
            case 7: F32_HALF(1, 7); break;
            case -1: F32_HALF(2, 1); break;
            case -3: F32_HALF(2, 3); break;
            case -5: F32_HALF(2, 5); break;
            default: F32_HALF(2, 7); break;
        }
    } else if (nv > 0) {
        switch ((nv <= 2 ? 2 : nv <= 4 ? 4 : 8) * (two ? -1 : 1)) {
            case 2: F32_LAUNCH(1, true, 2); break;
            case 4: F32_LAUNCH(1, true, 4); break;
            case 8: F32_LAUNCH(1, true, 8); break;
            case -2: F32_LAUNCH(2, true, 2); break;
            case -4: F32_LAUNCH(2, true, 4); break;
            default: F32_LAUNCH(2, true, 8); break;
        }
    } else if (two) {
        if (vec) F32_LAUNCH(2, true, 0);
        else F32_LAUNCH(2, false, 0);
    } else {
        if (vec) F32_LAUNCH(1, true, 0);
        else F32_LAUNCH(1, false, 0);
    }
#undef F32_LAUNCH
#undef F32_HALF
    return hipGetLastError() == hipSuccess ? RINA_OK : RINA_ERR_HIP;
}

bool mfma_ok(int qt, const float* x, int M, int K) {
    return M >= 16 && (qt == RINA_QT_Q4_0 || qt == RINA_QT_Q4_0F || qt == RINA_QT_GGML_Q2_K) && K % 32 == 0 &&
           (uintptr_t)x % 16 == 0;
}

// Matrix-core prompt matmul over up to 3 segments sharing x (one launch).
int gemm_mfma(const rina_linear_seg* segs, int nseg, int qt, const float* x, int M, int K, int epi, hipStream_t st) {
    MfmaArgs ma{};
    ma.g = GemmArgs{(const uint8_t*)segs[0].weight, epi == RINA_EPI_SWIGLU ? (const uint8_t*)segs[0].weight2 : nullptr,
                    x, segs[0].out, M, segs[0].N, K, qt, epi};
    ma.nseg = nseg;
    const bool two = epi == RINA_EPI_SWIGLU;
    // Q4 launches take 128-column tiles of eight waves (the x tile's split
    // and staging then serve twice the columns) when those tiles fill the
    // CUs in whole rounds, else 64-column tiles of four waves (q/k/v at M
    // 512: 384 wide tiles would leave half the CUs a second one); Q2_K
    // 64-column tiles
    auto count = [&](int bn) {
        int t = 0;
        for (int s = 0; s < nseg; s++) t += (segs[s].N + bn - 1) / bn;
        return t;
    };
    const bool half = (int64_t)count(64) * ((M + 63) / 64) < 2LL * rina_num_cus();   // 32-row tiles: more workgroups in flight
    const int64_t mtiles = half ? (M + 31) / 32 : (M + 63) / 64;
    const bool wide = qt != RINA_QT_GGML_Q2_K && mtiles * count(128) % rina_num_cus() == 0;
    const int BN = wide ? 128 : 64;
    int tiles = 0;
    for (int s = 0; s < 3; s++) {
        const int ss = s < nseg ? s : 0;
        ma.w[s] = (const uint8_t*)segs[ss].weight;
        ma.y[s] = segs[ss].out;
        ma.N[s] = segs[ss].N;
        ma.t0[s] = s < nseg ? tiles : 1 << 30;
        if (s < nseg) tiles += (segs[s].N + BN - 1) / BN;
    }
    ma.mt = half ? (M + 31) / 32 : (M + 63) / 64;
    ma.nt = tiles;
    // bytes the 8 L2s fetch for a split of x into 8 / xb parts and the
    // weights into xb parts: xb * (x bytes) + (8 / xb) * (weight bytes)
    const double xbytes = 4.0 * M * K;
    const double wbytes = (two ? 2.0 : 1.0) * BN * (double)tiles * K *
                          (qt == RINA_QT_Q4_0F ? 20.0 / 32 : qt == RINA_QT_GGML_Q2_K ? 84.0 / 256 : 18.0 / 32);
    int best = 1;
    for (int xb = 2; xb <= 8; xb *= 2)
        if (xb * xbytes + (8 / xb) * wbytes < best * xbytes + (8 / best) * wbytes) best = xb;
    ma.xb = best;
    ma.mpp = (ma.mt + 8 / best - 1) / (8 / best);
    ma.npp = (tiles + best - 1) / best;
    const dim3 g(8 * ma.mpp * ma.npp);
#define MFMA_LAUNCH(KN, F, NM) \
    do { if (half) hipLaunchKernelGGL((KN<F, NM, 32>), g, dim3(256), 0, st, ma); \
         else hipLaunchKernelGGL((KN<F, NM, 64>), g, dim3(256), 0, st, ma); } while (0)
    // Q4 weights: bf16 matrix cores on exact three-part splits of x; Q2_K
    // (weights d sc q - dmin m, not small integers): fp32 matrix cores
#define BF3_WN(F, NM, WN) \
    do { if (half) hipLaunchKernelGGL((gemm_bf3_kernel<F, NM, 32, WN>), g, dim3(128 * WN), 0, st, ma); \
         else hipLaunchKernelGGL((gemm_bf3_kernel<F, NM, 64, WN>), g, dim3(128 * WN), 0, st, ma); } while (0)
#define BF3_LAUNCH(F, NM) \
    do { if (wide) BF3_WN(F, NM, 4); else BF3_WN(F, NM, 2); } while (0)
    if (qt == RINA_QT_GGML_Q2_K) {
        if (two) MFMA_LAUNCH(gemm_mfma_kernel, FMT_Q2_K, 2);
        else MFMA_LAUNCH(gemm_mfma_kernel, FMT_Q2_K, 1);
    } else if (qt == RINA_QT_Q4_0F) {
        if (two) BF3_LAUNCH(FMT_Q4_0F, 2);
        else BF3_LAUNCH(FMT_Q4_0F, 1);
    } else {
        if (two) BF3_LAUNCH(FMT_Q4_0, 2);
        else BF3_LAUNCH(FMT_Q4_0, 1);
    }
#undef BF3_LAUNCH
#undef BF3_WN
#undef MFMA_LAUNCH
    return hipGetLastError() == hipSuccess ? RINA_OK : RINA_ERR_HIP;
}

int gemm_tiled(const rina_linear_seg& seg, int qt, const float* x, int M, int K, int epi, hipStream_t st) {
    // matrix cores for prompt-sized M and Q4 / Q2_K weights (K % 32 == 0, x
    // rows 16-byte aligned; weights 4-byte aligned)
    if (mfma_ok(qt, x, M, K)) return gemm_mfma(&seg, 1, qt, x, M, K, epi, st);
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

extern "C" int rina_hip_linear_fused_ex(const rina_linear_seg* segs, int nseg, int qt, const float* input, int M,
                                        int K, int epi, int pro, const float* nw, float eps, float* norm_out,
                                        void* stream) {
    if (!segs || nseg < 1 || nseg > kMaxDirectSegs || !input || M < 1 || K < 1) return RINA_ERR_ARG;
    if (!qt_supported(qt)) return RINA_ERR_QTYPE;
    if (epi < RINA_EPI_STORE || epi > RINA_EPI_SWIGLU) return RINA_ERR_ARG;
    if (pro < RINA_PRO_NONE || pro > RINA_PRO_LAYERNORM || (pro != RINA_PRO_NONE && !nw)) return RINA_ERR_ARG;
    if (norm_out && (pro == RINA_PRO_NONE || M != 1)) return RINA_ERR_ARG;
    if (epi == RINA_EPI_SWIGLU && nseg != 1) return RINA_ERR_ARG;
    if ((qt == RINA_QT_Q4_0 || qt == RINA_QT_Q4_0F) && (K % 32)) return RINA_ERR_SHAPE;
    for (int s = 0; s < nseg; s++) {
        if (!segs[s].weight || !segs[s].out || segs[s].N < 1) return RINA_ERR_ARG;
        if (epi == RINA_EPI_SWIGLU && !segs[s].weight2) return RINA_ERR_ARG;
        if ((uintptr_t)segs[s].weight % 4 || (segs[s].weight2 && (uintptr_t)segs[s].weight2 % 4)) return RINA_ERR_ARG;
    }
    hipStream_t st = as_stream(stream);
    int unit = qt == RINA_QT_GGML_Q2_K ? 16 : 32;
    int wpr = 1, cpl = 1;
    if (qt != RINA_QT_FP32 && K % unit == 0) split_row(K / unit, wpr, cpl);
    // direct kernel: any waves-per-row, up to kMaxDirectSegs segments; other
    // kernels: 3 segments per launch
    const bool direct = M == 1 && qt != RINA_QT_FP32 && direct_ok(fmt_of(qt), K) && (uintptr_t)input % 16 == 0;
    bool fused_pro = M == 1 && ((qt == RINA_QT_FP32 && K <= 16384) ||
                                (qt != RINA_QT_FP32 && (direct || (wpr == 1 && cpl == 1)) && (uintptr_t)input % 16 == 0 &&
                                 (uintptr_t)nw % 16 == 0));
    if (direct && norm_out && (uintptr_t)norm_out % 16) fused_pro = false;
    if (pro != RINA_PRO_NONE && (!fused_pro || (norm_out && !direct))) {
        // normalize first (into norm_out when given, else library scratch):
        // prompt rows, unusual shapes
        float* tmp = norm_out ? norm_out : (float*)rina_scratch((size_t)M * K * 4, as_stream(stream));
        if (!tmp) return RINA_ERR_HIP;
        int rc = pro == RINA_PRO_RMSNORM ? rina_hip_rms_norm(input, tmp, nw, M, K, eps, stream)
                                         : rina_hip_layer_norm(input, tmp, nw, M, K, eps, stream);
        if (rc) return rc;
        input = tmp;
        pro = RINA_PRO_NONE;
        norm_out = nullptr;
    }
    if (nseg > 3 && !direct) {   // the other kernels take 3 segments per launch
        for (int s0 = 0; s0 < nseg; s0 += 3) {
            int rc = rina_hip_linear_fused_ex(segs + s0, nseg - s0 < 3 ? nseg - s0 : 3, qt, input, M, K, epi, pro, nw,
                                              eps, nullptr, stream);
            if (rc) return rc;
        }
        return RINA_OK;
    }
    if (M > 1) {
        if (mfma_ok(qt, input, M, K)) return gemm_mfma(segs, nseg, qt, input, M, K, epi, st);   // nseg <= 3 here
        for (int s = 0; s < nseg; s++) {
            int rc = gemm_tiled(segs[s], qt, input, M, K, epi, st);
            if (rc) return rc;
        }
        return RINA_OK;
    }
    if (qt == RINA_QT_FP32) return gemv_f32(segs, nseg, input, K, epi, pro, nw, eps, st);
    if ((uintptr_t)input % 16) {   // register staging of x uses 16-byte loads
        for (int s = 0; s < nseg; s++) {
            int rc = gemm_tiled(segs[s], qt, input, M, K, epi, st);
            if (rc) return rc;
        }
        return RINA_OK;
    }
    return gemv_quant(segs, nseg, qt, input, K, epi, pro, nw, eps, norm_out, st);
}

extern "C" int rina_hip_linear_argmax(const rina_linear_seg* seg, int qt, const float* input, int K, int pro,
                                      const float* nw, float eps, void* keys, int max_keys, int* nkeys, void* stream) {
    if (!seg || !seg->weight || !seg->out || seg->N < 1 || !input || K < 1 || !keys || max_keys < 1 || !nkeys ||
        (uintptr_t)keys % 8)
        return RINA_ERR_ARG;
    if (qt != RINA_QT_FP32) return RINA_ERR_QTYPE;
    if (pro < RINA_PRO_NONE || pro > RINA_PRO_LAYERNORM || (pro != RINA_PRO_NONE && !nw)) return RINA_ERR_ARG;
    if (K > 16384) return RINA_ERR_SHAPE;
    return gemv_f32(seg, 1, input, K, RINA_EPI_STORE, pro, nw, eps, as_stream(stream), (unsigned long long*)keys,
                    max_keys, nkeys);
}

extern "C" int rina_hip_linear_fused(const rina_linear_seg* segs, int nseg, int qt, const float* input, int M, int K,
                                     int epi, int pro, const float* nw, float eps, void* stream) {
    return rina_hip_linear_fused_ex(segs, nseg, qt, input, M, K, epi, pro, nw, eps, nullptr, stream);
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
        dst = (float*)rina_scratch((size_t)M * N * 4, st);
        if (!dst) return RINA_ERR_HIP;
    }
    rina_linear_seg seg{weight, nullptr, dst, N};
    int rc = rina_hip_linear_fused(&seg, 1, qt, input, M, K, RINA_EPI_STORE, RINA_PRO_NONE, nullptr, 0.f, stream);
    if (rc) return rc;
    if (alias && hipMemcpyAsync(output, dst, (size_t)M * N * 4, hipMemcpyDeviceToDevice, st) != hipSuccess)
        return RINA_ERR_HIP;
    return RINA_OK;
}
