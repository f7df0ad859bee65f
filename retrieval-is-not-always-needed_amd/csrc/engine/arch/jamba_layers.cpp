// RINA Jamba hybrid layers on the gfx950 C-ABI, with the reference's tensor
// names:
//   InertiaWave SSM (arch/ssm/rina_ssm_layer.cu:90-126): x = LN(h, ln1);
//     cq = LN(W_dq x, q_norm); mem_k = W_mem[k] cq, dec_k = sigmoid(W_decay[k]
//     cq) (k < ssm_steps); 3-step aggregation and the log-space scan;
//     h += W_out [x | sf]; MLP.
//   RINA-MLA (arch/mla/rina_mla_layer.cu:65-98): x = LN(h, ln1);
//     cq = LN(W_dqkv x, q_norm); q = W_uq cq, k = W_uk cq, v = W_k2v k;
//     qr = HF-RoPE(W_qr x), kr = HF-RoPE(W_kr x); causal attention with
//     query [q | qr], key [k | kr], scale 1/sqrt(dh + dhr); h += c_proj o; MLP.
//   MLP: h += W2 (SiLU(W1 LN(h, ln2)) * W3 LN(h, ln2)).
// The reference layers keep no state (every step recomputes the whole
// sequence, tests/test_infer.cu:58-80).  Here the SSM layer keeps its scan
// state and the RINA-MLA layer its fp32 K/V rows in device memory, advanced
// one position per token with the reference's per-position operations, so a
// decode step equals the full recompute.  A host-position call at
// start_pos 0 restarts the scan; calls must continue the sequence in order.
// A prompt (T > 1 rows at host positions) runs its matvecs as T-row
// matrix products, the SSM scan over all T positions in one launch
// (rina_hip_ssm_scan), and the RINA-MLA attention position by position
// (each row appends its K/V, then attends to the rows before it), with the
// rows' intermediates in ForwardBuffers::mla (workspace_per_token floats
// per row).
#include <algorithm>
#include <cstdio>
#include <string>
#include "core/buffer.h"
#include "core/config.h"
#include "core/layer.h"
#include "core/tensor.h"
#include "rina_hip.h"

namespace {

std::string tn(int l, const char* c, const char* p) {
    char b[160];
    snprintf(b, sizeof b, "transformer.h.%d.%s.%s", l, c, p);
    return b;
}

// Tensor lookup with the element count the config implies (the kernels
// index by the config, so a smaller tensor would be read past its end).
struct Loader {
    const TensorMap& w;
    int l;
    bool ok = true;
    QuantType qt = QuantType::FP32;
    bool first = true;
    const void* lin(const char* c, const char* p, int64_t rows, int64_t cols) {
        const WeightTensor* t = w.get(tn(l, c, p));
        if (!elems_are(t, rows * cols)) { ok = false; return t ? t->data : nullptr; }
        if (first) { qt = t->quant_type; first = false; }
        else if (t->quant_type != qt) ok = false;       // one quant type per layer
        return t->data;
    }
    // n > 0: exactly n values; n < 0: at least -n values (RoPE tables)
    const float* f32(const char* c, const char* p, int64_t n, bool required = true) {
        const WeightTensor* t = w.get(tn(l, c, p));
        if (!t) { if (required) ok = false; return nullptr; }
        if (t->quant_type != QuantType::FP32 || !(n > 0 ? elems_are(t, n) : elems_at_least(t, -n))) ok = false;
        return (const float*)t->data;
    }
};

template <typename T>
bool dev_alloc(T** p, size_t n) {
    if (hipMalloc((void**)p, n * sizeof(T)) != hipSuccess) { *p = nullptr; return false; }
    return hipMemset(*p, 0, n * sizeof(T)) == hipSuccess;
}

struct MLPPart {
    const void *w1 = nullptr, *w2 = nullptr, *w3 = nullptr;
    const float *ln2 = nullptr;
    int hd = 0;
    // h[M, d] += MLP(h) for M rows (b.g holds M rows of hd)
    int run(float* ht, ForwardBuffers& b, int d, int qt, hipStream_t s, int M = 1) const {
        int rc;
        rina_linear_seg up{w1, w3, b.g, hd};
        if ((rc = rina_hip_linear_fused(&up, 1, qt, ht, M, d, RINA_EPI_SWIGLU, RINA_PRO_LAYERNORM, ln2, 1e-5f, s)))
            return rc;
        rina_linear_seg down{w2, nullptr, ht, d};
        return rina_hip_linear_fused(&down, 1, qt, b.g, M, hd, RINA_EPI_ADD, RINA_PRO_NONE, nullptr, 0.f, s);
    }
};

struct SSMImpl {
    int d = 0, H = 0, dh = 0, dc = 0, steps = 0;
    int qt = 0;
    const float *ln1 = nullptr, *q_norm = nullptr;
    const void *w_dq = nullptr, *w_mem[3] = {}, *w_decay[3] = {}, *w_out = nullptr;
    MLPPart mlp;
    float *lcs = nullptr, *wcs = nullptr;      // scan state [H*dh]
    float* scratch = nullptr;                  // x2 [d + H*dh] | cq [dc] | mem [3*H*dh] | dec [3*H]
    bool fused = true;                         // rina_hip_ssm_proj_step takes this layer's shape

    ~SSMImpl() {
        if (lcs) (void)hipFree(lcs);
        if (wcs) (void)hipFree(wcs);
        if (scratch) (void)hipFree(scratch);
    }

    bool init(const ModelConfig& cfg, const TensorMap& w, int l) {
        d = cfg.dim; H = cfg.n_heads; dh = cfg.head_dim;
        dc = cfg.d_c > 0 ? cfg.d_c : 160;
        steps = cfg.ssm_steps > 0 ? cfg.ssm_steps : 3;
        if (steps > 3) return false;
        const WeightTensor* t1 = w.get(tn(l, "mlp", "w1.weight"));
        if (!t1 || t1->n_dim < 2) return false;
        mlp.hd = t1->shape[0];
        Loader L{w, l};
        w_dq = L.lin("path", "w_dq.weight", dc, d);
        for (int k = 0; k < steps; k++) {
            char b1[48], b2[48];
            snprintf(b1, sizeof b1, "w_mem.%d.weight", k);
            snprintf(b2, sizeof b2, "w_decay.%d.weight", k);
            w_mem[k] = L.lin("path", b1, (int64_t)H * dh, dc);
            w_decay[k] = L.lin("path", b2, H, dc);
        }
        w_out = L.lin("path", "w_out.weight", d, (int64_t)d + H * dh);
        mlp.w1 = L.lin("mlp", "w1.weight", mlp.hd, d);
        mlp.w2 = L.lin("mlp", "w2.weight", d, mlp.hd);
        mlp.w3 = L.lin("mlp", "w3.weight", mlp.hd, d);
        q_norm = L.f32("path", "q_norm.weight", dc);
        ln1 = L.f32("ln1", "weight", d);
        mlp.ln2 = L.f32("ln2", "weight", d);
        if (!L.ok) return false;
        qt = (int)L.qt;
        return dev_alloc(&lcs, (size_t)H * dh) && dev_alloc(&wcs, (size_t)H * dh) &&
               dev_alloc(&scratch, (size_t)d + H * dh + dc + 3 * H * dh + 3 * H);
    }

    // prompt rows: xln [T][d] | x2 [T][d + H*dh] | cq [T][dc] | mem [steps][T][H*dh] | dec [steps][T][H]
    int rows_per_token() const { return 2 * d + H * dh + dc + steps * (H * dh + H); }

    int forward_rows(float* h, ForwardBuffers& b, int T, hipStream_t s) {
        const int start_pos = b.kv_cache.start_pos;
        const int xw = d + H * dh;
        float* xln = b.mla;
        float* x2 = xln + (size_t)T * d;
        float* cq = x2 + (size_t)T * xw;
        float* mem = cq + (size_t)T * dc;
        float* dec = mem + (size_t)steps * T * H * dh;
        int rc;
#define CK(x) do { if ((rc = (x)) != RINA_OK) return rc; } while (0)
        // x = LN(h, ln1) (:93-96), kept as the first d columns of W_out's input rows
        CK(rina_hip_layer_norm(h, xln, ln1, T, d, 1e-5f, s));
        if (hipMemcpy2DAsync(x2, sizeof(float) * xw, xln, sizeof(float) * d, sizeof(float) * d, T,
                             hipMemcpyDeviceToDevice, s) != hipSuccess)
            return RINA_ERR_HIP;
        rina_linear_seg sq{w_dq, nullptr, cq, dc};
        CK(rina_hip_linear_fused(&sq, 1, qt, xln, T, d, RINA_EPI_STORE, RINA_PRO_NONE, nullptr, 0.f, s));
        // LN(cq, q_norm) and the memory / decay projections of every row (:97-101)
        rina_linear_seg sp[6];
        for (int k = 0; k < steps; k++) {
            sp[k] = {w_mem[k], nullptr, mem + (size_t)k * T * H * dh, H * dh};
            sp[steps + k] = {w_decay[k], nullptr, dec + (size_t)k * T * H, H};
        }
        CK(rina_hip_linear_fused(sp, 2 * steps, qt, cq, T, dc, RINA_EPI_STORE, RINA_PRO_LAYERNORM, q_norm, 1e-5f, s));
        // the scan over the T positions (:102-109), sf into the last H*dh columns of x2
        CK(rina_hip_ssm_scan(mem, dec, steps, H, dh, T, lcs, wcs, x2 + d, xw, start_pos == 0 ? 1 : 0, s));
        rina_linear_seg so{w_out, nullptr, h, d};
        CK(rina_hip_linear_fused(&so, 1, qt, x2, T, xw, RINA_EPI_ADD, RINA_PRO_NONE, nullptr, 0.f, s));
        CK(mlp.run(h, b, d, qt, s, T));
#undef CK
        return RINA_OK;
    }

    int forward(float* h, ForwardBuffers& b, int T, hipStream_t s) {
        if (T > 1 && !b.d_pos && b.mla) return forward_rows(h, b, T, s);
        const int start_pos = b.kv_cache.start_pos;
        float* x2 = scratch;
        float* cq = x2 + d + H * dh;
        float* mem = cq + dc;
        float* dec = mem + 3 * H * dh;
        int rc;
#define CK(x) do { if ((rc = (x)) != RINA_OK) return rc; } while (0)
        for (int t = 0; t < T; t++) {
            float* ht = h + (size_t)t * d;
            // x = LN(h, ln1) as W_dq's prologue; the launch also stores x for W_out (:93-96)
            rina_linear_seg sq{w_dq, nullptr, cq, dc};
            CK(rina_hip_linear_fused_ex(&sq, 1, qt, ht, 1, d, RINA_EPI_STORE, RINA_PRO_LAYERNORM, ln1, 1e-5f, x2, s));
            const int reset = (!b.d_pos && start_pos == 0 && t == 0) ? 1 : 0;
            // LN(cq, q_norm), the memory and decay projections and the scan
            // step (:97-109) in one launch where the kernel takes the shape
            rc = fused ? rina_hip_ssm_proj_step(cq, q_norm, 1e-5f, w_mem, w_decay, qt, steps, H, dh, dc, lcs, wcs,
                                                x2 + d, reset, s)
                       : RINA_ERR_SHAPE;
            if (rc == RINA_ERR_QTYPE || rc == RINA_ERR_SHAPE) {
                fused = false;
                // the projections share LN(cq, q_norm): one launch, then the step
                rina_linear_seg sp[6];
                for (int k = 0; k < steps; k++) {
                    sp[k] = {w_mem[k], nullptr, mem + (size_t)k * H * dh, H * dh};
                    sp[steps + k] = {w_decay[k], nullptr, dec + (size_t)k * H, H};
                }
                CK(rina_hip_linear_fused(sp, 2 * steps, qt, cq, 1, dc, RINA_EPI_STORE, RINA_PRO_LAYERNORM, q_norm,
                                         1e-5f, s));
                CK(rina_hip_ssm_step(mem, dec, steps, H, dh, lcs, wcs, x2 + d, reset, s));
            } else if (rc != RINA_OK) {
                return rc;
            }
            rina_linear_seg so{w_out, nullptr, ht, d};
            CK(rina_hip_linear_fused(&so, 1, qt, x2, 1, d + H * dh, RINA_EPI_ADD, RINA_PRO_NONE, nullptr, 0.f, s));
            CK(mlp.run(ht, b, d, qt, s));
        }
#undef CK
        return RINA_OK;
    }
};

struct RMLAImpl {
    int d = 0, H = 0, Hkv = 0, dh = 0, dhr = 0, dc = 0, max_seq = 0;
    int qt = 0;
    const float *ln1 = nullptr, *q_norm = nullptr;
    const float *rqc = nullptr, *rqs = nullptr, *rkc = nullptr, *rks = nullptr;
    const void *w_dqkv = nullptr, *w_uq = nullptr, *w_uk = nullptr, *w_k2v = nullptr, *w_qr = nullptr,
               *w_kr = nullptr, *c_proj = nullptr;
    MLPPart mlp;
    // K / V cache: fp32 K [max_seq][Hkv][dh+dhr] and V [max_seq][Hkv][dh]
    // (kv_mode RINA_KV_FP32), or the q2k_q1v form: q2_1 key content, fp32
    // RoPE part (kr), q1_0 values (rina_hip_dq_decode_attention_kv)
    int kv_mode = RINA_KV_FP32;
    void *ck = nullptr, *cv = nullptr;
    float* ckr = nullptr;
    float* scratch = nullptr;                  // cq | qr | kr | q | k | v | att
    void* ws = nullptr;
    size_t ws_bytes = 0;

    ~RMLAImpl() {
        if (ck) (void)hipFree(ck);
        if (cv) (void)hipFree(cv);
        if (ckr) (void)hipFree(ckr);
        if (scratch) (void)hipFree(scratch);
        if (ws) (void)hipFree(ws);
    }

    bool init(const ModelConfig& cfg, const TensorMap& w, int l) {
        d = cfg.dim; H = cfg.n_heads; Hkv = cfg.n_kv_heads; dh = cfg.head_dim;
        dhr = cfg.d_h_r > 0 ? cfg.d_h_r : 32;
        dc = cfg.d_c > 0 ? cfg.d_c : 160;
        max_seq = cfg.max_seq_len > 0 ? cfg.max_seq_len : 512;
        if (Hkv <= 0 || H % Hkv) return false;
        const WeightTensor* t1 = w.get(tn(l, "mlp", "w1.weight"));
        if (!t1 || t1->n_dim < 2) return false;
        mlp.hd = t1->shape[0];
        Loader L{w, l};
        w_dqkv = L.lin("path", "w_dqkv.weight", dc, d);
        w_qr = L.lin("path", "w_qr.weight", (int64_t)H * dhr, d);
        w_kr = L.lin("path", "w_kr.weight", (int64_t)Hkv * dhr, d);
        w_uq = L.lin("path", "w_uq.weight", (int64_t)H * dh, dc);
        w_uk = L.lin("path", "w_uk.weight", (int64_t)Hkv * dh, dc);
        w_k2v = L.lin("path", "w_k2v.weight", (int64_t)Hkv * dh, (int64_t)Hkv * dh);
        c_proj = L.lin("path", "c_proj.weight", d, (int64_t)H * dh);
        mlp.w1 = L.lin("mlp", "w1.weight", mlp.hd, d);
        mlp.w2 = L.lin("mlp", "w2.weight", d, mlp.hd);
        mlp.w3 = L.lin("mlp", "w3.weight", mlp.hd, d);
        q_norm = L.f32("path", "q_norm.weight", dc);
        ln1 = L.f32("ln1", "weight", d);
        mlp.ln2 = L.f32("ln2", "weight", d);
        const int64_t rope_n = -(int64_t)max_seq * (dhr / 2);
        rqc = L.f32("path", "rope_q.cos", rope_n, false); rqs = L.f32("path", "rope_q.sin", rope_n, false);
        rkc = L.f32("path", "rope.cos", rope_n, false); rks = L.f32("path", "rope.sin", rope_n, false);
        if (!L.ok) return false;
        qt = (int)L.qt;
        ws_bytes = rina_hip_dq_attention_workspace(H, dh + dhr, max_seq);
        const size_t sc = (size_t)dc + H * dhr + Hkv * dhr + H * dh + 2 * Hkv * dh + H * dh;
        // kv_quant_mode applies to GQA caches only; the reference's RINA-MLA
        // layer keeps fp32 rows whatever it says (rina_mla_layer.cu:65-98).
        // The packed q2 K / q1 V cache is the engine's own opt-in key,
        // rina_mla_kv_mode "q2k_q1v" (queries and the current position stay
        // fp32; only earlier positions are read through their packs)
        const std::string& km = cfg.rina_mla_kv_mode;
        int mode;
        if (km.empty() || km == "fp32") mode = RINA_KV_FP32;
        else if (km == "q2k_q1v") mode = RINA_KV_Q2K_Q1V;
        else return false;
        kv_mode = mode;
        const size_t kb = rina_hip_dq_kv_region_bytes(mode, 0, max_seq, Hkv, dh, dhr, dh);
        const size_t vb = rina_hip_dq_kv_region_bytes(mode, 1, max_seq, Hkv, dh, dhr, dh);
        const size_t rb = rina_hip_dq_kv_region_bytes(mode, 2, max_seq, Hkv, dh, dhr, dh);
        if (!kb || !vb) return false;
        return dev_alloc((uint8_t**)&ck, kb) && dev_alloc((uint8_t**)&cv, vb) &&
               (!rb || dev_alloc((uint8_t**)&ckr, rb)) && dev_alloc(&scratch, sc) && dev_alloc((uint8_t**)&ws, ws_bytes);
    }

    // prompt rows: cq [T][dc] | qr [T][H*dhr] | kr [T][Hkv*dhr] | q [T][H*dh] | k, v [T][Hkv*dh] | att [T][H*dh]
    // | the fp32-cache prompt attention's rows (rina_hip_dq_prompt_workspace per row)
    int attn_rows_per_token() const { return 2 * (H + Hkv) * (dh + dhr); }
    int rows_per_token() const {
        return dc + H * dhr + Hkv * dhr + 2 * H * dh + 2 * Hkv * dh + attn_rows_per_token();
    }

    int forward_rows(float* h, ForwardBuffers& b, int T, hipStream_t s) {
        const int start_pos = b.kv_cache.start_pos;
        float* cq = b.mla;
        float* qr = cq + (size_t)T * dc;
        float* kr = qr + (size_t)T * H * dhr;
        float* q = kr + (size_t)T * Hkv * dhr;
        float* k = q + (size_t)T * H * dh;
        float* v = k + (size_t)T * Hkv * dh;
        float* att = v + (size_t)T * Hkv * dh;
        int rc;
#define CK(x) do { if ((rc = (x)) != RINA_OK) return rc; } while (0)
        rina_linear_seg s1[3] = {{w_dqkv, nullptr, cq, dc}, {w_qr, nullptr, qr, H * dhr}, {w_kr, nullptr, kr, Hkv * dhr}};
        CK(rina_hip_linear_fused(s1, 3, qt, h, T, d, RINA_EPI_STORE, RINA_PRO_LAYERNORM, ln1, 1e-5f, s));
        rina_linear_seg s2[2] = {{w_uq, nullptr, q, H * dh}, {w_uk, nullptr, k, Hkv * dh}};
        CK(rina_hip_linear_fused(s2, 2, qt, cq, T, dc, RINA_EPI_STORE, RINA_PRO_LAYERNORM, q_norm, 1e-5f, s));
        rina_linear_seg s3{w_k2v, nullptr, v, Hkv * dh};
        CK(rina_hip_linear_fused(&s3, 1, qt, k, T, Hkv * dh, RINA_EPI_STORE, RINA_PRO_NONE, nullptr, 0.f, s));
        // causal attention (:78-86): row t appends its K / V at start_pos + t and
        // attends to positions <= it.  One call appends every row, then each
        // row reads the rows before it through the cache; shapes it does not
        // take: fp32 caches from position 0 as one causal pass over the
        // expanded rows, else row by row
        bool batched = false;
        rc = rina_hip_dq_prompt_attention_kv(q, qr, k, kr, v, rqc, rqs, rkc, rks, kv_mode, ck, cv, ckr, H, Hkv, dh, dhr,
                                             dh, start_pos, T, max_seq, att, s);
        if (rc != RINA_OK && rc != RINA_ERR_SHAPE) return rc;   // a shape it does not take launches nothing
        batched = rc == RINA_OK;
        if (!batched && kv_mode == RINA_KV_FP32 && start_pos == 0) {
            float* aws = att + (size_t)T * H * dh;
            const size_t need = rina_hip_dq_prompt_workspace(T, H, Hkv, dh, dhr, dh);
            if (need && need <= sizeof(float) * (size_t)T * attn_rows_per_token() && (uintptr_t)aws % 16 == 0) {
                rc = rina_hip_dq_prompt_attention(q, qr, k, kr, v, rqc, rqs, rkc, rks, (float*)ck, (float*)cv, H, Hkv,
                                                  dh, dhr, dh, T, max_seq, att, aws, need, s);
                if (rc != RINA_OK && rc != RINA_ERR_SHAPE) return rc;   // a shape it does not take launches nothing
                batched = rc == RINA_OK;
            }
        }
        for (int t = 0; t < T && !batched; t++)
            CK(rina_hip_dq_decode_attention_kv(q + (size_t)t * H * dh, qr + (size_t)t * H * dhr, k + (size_t)t * Hkv * dh,
                                               kr + (size_t)t * Hkv * dhr, v + (size_t)t * Hkv * dh, rqc, rqs, rkc, rks,
                                               kv_mode, ck, cv, ckr, H, Hkv, dh, dhr, dh, start_pos + t, nullptr,
                                               max_seq, att + (size_t)t * H * dh, ws, ws_bytes, s));
        rina_linear_seg so{c_proj, nullptr, h, d};
        CK(rina_hip_linear_fused(&so, 1, qt, att, T, H * dh, RINA_EPI_ADD, RINA_PRO_NONE, nullptr, 0.f, s));
        CK(mlp.run(h, b, d, qt, s, T));
#undef CK
        return RINA_OK;
    }

    int forward(float* h, ForwardBuffers& b, int T, hipStream_t s) {
        if (T > 1 && !b.d_pos && b.mla) return forward_rows(h, b, T, s);
        const int start_pos = b.kv_cache.start_pos;
        float* cq = scratch;
        float* qr = cq + dc;
        float* kr = qr + H * dhr;
        float* q = kr + Hkv * dhr;
        float* k = q + H * dh;
        float* v = k + Hkv * dh;
        float* att = v + Hkv * dh;
        int rc;
#define CK(x) do { if ((rc = (x)) != RINA_OK) return rc; } while (0)
        for (int t = 0; t < T; t++) {
            float* ht = h + (size_t)t * d;
            // W_dqkv, W_qr, W_kr share x = LN(h, ln1): one launch with the norm as prologue
            rina_linear_seg s1[3] = {{w_dqkv, nullptr, cq, dc}, {w_qr, nullptr, qr, H * dhr}, {w_kr, nullptr, kr, Hkv * dhr}};
            CK(rina_hip_linear_fused(s1, 3, qt, ht, 1, d, RINA_EPI_STORE, RINA_PRO_LAYERNORM, ln1, 1e-5f, s));
            rina_linear_seg s2[2] = {{w_uq, nullptr, q, H * dh}, {w_uk, nullptr, k, Hkv * dh}};
            CK(rina_hip_linear_fused(s2, 2, qt, cq, 1, dc, RINA_EPI_STORE, RINA_PRO_LAYERNORM, q_norm, 1e-5f, s));
            rina_linear_seg s3{w_k2v, nullptr, v, Hkv * dh};
            CK(rina_hip_linear_fused(&s3, 1, qt, k, 1, Hkv * dh, RINA_EPI_STORE, RINA_PRO_NONE, nullptr, 0.f, s));
            CK(rina_hip_dq_decode_attention_kv(q, qr, k, kr, v, rqc, rqs, rkc, rks, kv_mode, ck, cv, ckr, H, Hkv, dh,
                                               dhr, dh, start_pos + t, b.d_pos, max_seq, att, ws, ws_bytes, s));
            rina_linear_seg so{c_proj, nullptr, ht, d};
            CK(rina_hip_linear_fused(&so, 1, qt, att, 1, H * dh, RINA_EPI_ADD, RINA_PRO_NONE, nullptr, 0.f, s));
            CK(mlp.run(ht, b, d, qt, s));
        }
#undef CK
        return RINA_OK;
    }
};

template <typename Impl>
bool v_init(void* self, const ModelConfig& c, const TensorMap& w, int l) { return ((Impl*)self)->init(c, w, l); }
template <typename Impl>
void v_forward(void* self, float* h, ForwardBuffers& b, int B, int T, hipStream_t s) {
    (void)B;
    b.fail(((Impl*)self)->forward(h, b, T, s));
}
// floats per prompt row the layer needs in ForwardBuffers::mla
template <typename Impl>
int v_ws(void* self, int, int, int) { return ((Impl*)self)->rows_per_token(); }
template <typename Impl>
void v_destroy(void* self) { delete (Impl*)self; }

const LayerVTable kSSMVTable = {v_init<SSMImpl>, v_forward<SSMImpl>, layer_no_backward, v_ws<SSMImpl>, layer_no_saved,
                                v_destroy<SSMImpl>};
const LayerVTable kRMLAVTable = {v_init<RMLAImpl>, v_forward<RMLAImpl>, layer_no_backward, v_ws<RMLAImpl>,
                                 layer_no_saved, v_destroy<RMLAImpl>};

}  // namespace

Layer create_ssm_layer() {
    Layer l;
    l.impl = new SSMImpl();
    l.vtab = &kSSMVTable;
    return l;
}

Layer create_rina_mla_layer() {
    Layer l;
    l.impl = new RMLAImpl();
    l.vtab = &kRMLAVTable;
    return l;
}
