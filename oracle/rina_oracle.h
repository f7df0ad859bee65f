/*
 * rina_oracle.h — CPU restatement of the RINA engine's decode-step hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the
 * MI355X HIP path: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  The product never links or calls it.
 *
 * Every function names the reference file:line it restates (paths are
 * relative to the reference repository root, rina-engine/src/...).
 * Arithmetic follows the reference's per-output loop order.  Where nvcc's
 * default --fmad=true would contract `sum += a*b` into an FMA, the oracle
 * writes fmaf() explicitly and is built with -ffp-contract=off, so the
 * rounding sequence is pinned independent of the host compiler.
 *
 * Pinning (how each function is checked, see tests/test_oracle_*.py):
 *   fp16 conversion        exhaustive vs numpy float16 (RNE) over all f16
 *                          values and edge cases; truncating variant vs
 *                          closed form.
 *   weight packers         known answers of rina-engine/tests/test_layers.cu
 *                          (0xEE -> 7, 0x77 -> 0), round-trip bound
 *                          |deq - x| <= scale/2, the 0.49999997f edge.
 *   q4 / q4f / fp32 matvec brute force in float64 (numpy) + the
 *                          test_linear_q4.cu shapes.
 *   Q2_K dequant           independent numpy bit-twiddling restatement of
 *                          the three in-repo statements; exact in fp32.
 *   KV packers             closed forms (numpy restatement), invariants.
 *   attention              float64 textbook softmax; single-key and
 *                          identical-keys invariants.
 *   glue / model           float64 numpy restatement on tiny shapes.
 */
#ifndef RINA_ORACLE_H
#define RINA_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* QuantType ids (rina-engine/src/core/quant.h:9-14) */
enum {
    ORC_Q2_1 = 1, ORC_Q1_0 = 2, ORC_Q4_0 = 5, ORC_FP32 = 6, ORC_Q4_0F = 7,
    ORC_GGML_Q2_K = 10
};

/* KV cache modes (rina-engine/src/core/buffer.h:49, buffer.cpp:104-113) */
enum { ORC_KV_FP32 = 0, ORC_KV_Q8 = 1, ORC_KV_Q4 = 2, ORC_KV_Q4K_Q2V = 3,
       ORC_KV_Q2 = 4, ORC_KV_Q2K_Q1V = 5 };

/* KV block formats for orc_kv_quantize / orc_kv_dequant */
enum { ORC_KVF_Q8_0 = 1, ORC_KVF_Q4_0 = 2, ORC_KVF_Q2_1 = 3, ORC_KVF_Q1_0 = 4 };

/* ---- fp16 ---------------------------------------------------------- */
uint16_t orc_f32_to_f16(float f);        /* IEEE RNE with subnormals (__float2half) */
uint16_t orc_f32_to_f16_trunc(float f);  /* loader_hf.cpp:208-216 truncating variant */
float    orc_f16_to_f32(uint16_t h);

/* ---- weight formats ------------------------------------------------ */
size_t orc_quantized_size(int64_t n_elems, int qt);     /* core/quant.h:75-86 */
void orc_pack_q4_0(const float* x, int64_t n, uint8_t* out);     /* tools/q4_pack.py:11-23,71-92 */
void orc_pack_q4_0f(const float* x, int64_t n, uint8_t* out);    /* tools/q4_pack.py:95-118 */
void orc_pack_q4_0_hf(const float* x, int64_t n, uint8_t* out);  /* src/loader_hf.cpp:196-230 */
/* dequantize n elements of a weight tensor (flat element order) to fp32 */
void orc_dequant_weights(const void* w, int qt, int64_t n, float* out);

/* ---- matvec -------------------------------------------------------- */
/* out[M,N] = in[M,K] . W[N,K]^T, the dispatch of ops/linear.cu:140-167.
 * nthreads <= 0 picks the host core count.  Row results are independent of
 * the thread count. */
int orc_linear(const void* w, int qt, const float* in, float* out,
               int M, int N, int K, int nthreads);

/* ---- KV cache block formats --------------------------------------- */
int  orc_kv_block_bytes(int fmt);   /* 34 / 18 / 10 / 6 */
void orc_kv_quantize(int fmt, const float* in, void* out, int64_t n);
void orc_kv_dequant(int fmt, const void* in, float* out, int64_t n);
void orc_kv_mode_formats(int mode, int* kfmt, int* vfmt);

/* ---- glue ---------------------------------------------------------- */
void orc_rms_norm(float* x, const float* w, int n, int d, float eps);    /* ops/rms_norm.cu:5-29 */
void orc_layer_norm(float* x, const float* w, int n, int d, float eps);  /* kernels/pytorch_ln_kernel.cu:4-35 */
void orc_rope_neox(float* x, const float* cos_t, const float* sin_t,
                   int T, int H, int d, int start_pos);                 /* ops/rope.cu:125-149 */
void orc_rope_hf(float* x, const float* cos_t, const float* sin_t,
                 int T, int H, int d, int start_pos);                   /* ops/rope.cu:212-234 */
void orc_embedding(const void* w, int qt, const int* ids, float* out, int n, int d); /* ops/embedding.cu:6-230 */
void orc_silu_mul(float* o, const float* g, const float* u, int n);     /* ops/silu_mul.cu:5-8 */
void orc_add(float* c, const float* a, const float* b, int n);          /* ops/saxpy.cu:10-13 */
void orc_saxpy(float* d, const float* s, float p, int n);               /* ops/saxpy.cu:5-8 */
int  orc_argmax(const float* x, int n);                                 /* main.cpp:139-146 */

/* ---- attention ----------------------------------------------------- */
/* Causal single-head attention of the online form in
 * kernels/flash_fp32.cu:12-94 for query rows [q0, q0+nq) over keys
 * [0, q0+i] of K[T,dq] / V[T,dh] (rows of one head, row stride ldk/ldv).
 * o receives nq rows of dh floats (row stride ldo). */
void orc_attn_rows(const float* q, int ldq, const float* k, int ldk,
                   const float* v, int ldv, float* o, int ldo,
                   int q0, int nq, int dq, int dh);

/* Decode/prefill attention of GQAImpl::forward (arch/gqa/gqa_layer.cu:155-270)
 * for one layer: queries q[T, H*dh] at positions start_pos..start_pos+T-1;
 * keys/values [0,start_pos) come from the layer's cache region (mode 0:
 * fp32 k_cache/v_cache [max_seq, Hkv*dh]; mode>0: quantized blocks at
 * kq/vq), keys [start_pos, start_pos+T) from kcur/vcur [T, Hkv*dh] fp32.
 * pre_rope: cached K is stored before RoPE and rotated on read with the
 * k tables.  out[T, H*dh]. */
void orc_gqa_attention(const float* q, const float* kcur, const float* vcur,
                       const float* k_cache, const float* v_cache,
                       const uint8_t* kq, const uint8_t* vq, int mode, int pre_rope,
                       const float* rope_k_cos, const float* rope_k_sin,
                       int T, int start_pos, int H, int Hkv, int dh, float* out);

/* ---- GQA (Llama-shaped) model -------------------------------------- */
typedef struct {
    const void* w_q; int qt_q;
    const void* w_k; int qt_k;
    const void* w_v; int qt_v;
    const void* w_o; int qt_o;
    const void* w1;  int qt_1;
    const void* w2;  int qt_2;
    const void* w3;  int qt_3;
    const float* ln1; const float* ln2;
    const float* rope_q_cos; const float* rope_q_sin;
    const float* rope_k_cos; const float* rope_k_sin;
} orc_gqa_layer_w;

typedef struct {
    int dim, n_layers, n_heads, n_kv_heads, head_dim, hidden, vocab, max_seq;
    int use_rms_norm;   /* cfg.name contains "llama" (gqa_layer.cu:90) */
    int kv_mode;        /* 0..5 */
    int pre_rope;
    int nthreads;
    const void* wte; int qt_wte;
    const float* ln_f;
    const void* lm_head; int qt_lm;   /* NULL -> tied to wte */
    const orc_gqa_layer_w* layers;
} orc_gqa_cfg;

typedef struct orc_gqa orc_gqa;
orc_gqa* orc_gqa_create(const orc_gqa_cfg* cfg);
void     orc_gqa_destroy(orc_gqa* m);
/* Inference::forward of infer/infer_gqa.cpp:75-105.  logits: [T, vocab]
 * (only the last row when last_only != 0). */
int      orc_gqa_forward(orc_gqa* m, const int* ids, int T, int start_pos,
                         float* logits, int last_only);
/* raw access to the oracle's cache (mode 0: float data; mode>0: bytes) */
void*    orc_gqa_cache(orc_gqa* m, int layer, int which_v, size_t* bytes);
/* fp32 K/V of the last forward's tokens for one layer (post-RoPE unless pre_rope) */
const float* orc_gqa_last_kv(orc_gqa* m, int layer, int which_v);
/* main.cpp:666-690 greedy loop: prefill then steps-1 decodes; writes steps ids */
int      orc_gqa_generate(orc_gqa* m, const int* prompt, int n_prompt, int steps, int* out_ids);

/* ---- DeepSeek MLA + MoE model ---------------------------------------- */
/* Router top-k of deepseek_mla_layer.cu:310-326: softmax over E logits
 * (max-subtracted expf, serial fp32 sum, one reciprocal), then insertion
 * top-k keeping topw ascending (strict ">": the earlier expert wins ties).
 * ids/probs in that ascending order; unfilled slots get id -1. */
void orc_moe_topk(const float* logits, int E, int k, int* ids, float* probs);

typedef struct {
    const void* w_q; int qt_q;          /* [H*(nope+rope), d]; row order [H*nope | H*rope] */
    const void* w_kv_a; int qt_kv_a;    /* [dc+rope, d]; row order [c_kv | k_pe] */
    const float* k_norm;                /* [dc] */
    const void* w_kv_b; int qt_kv_b;    /* [H*(nope+v), dc]; row order [H*nope | H*v] */
    const void* w_o; int qt_o;          /* [d, H*v] */
    const float* ln1; const float* ln2;
    const float* rope_cos; const float* rope_sin;   /* [max_pos][rope/2] (attn.rope_q) */
    int is_moe;
    const void* w1; int qt_1;           /* dense SwiGLU [hidden, d] */
    const void* w2; int qt_2;           /* [d, hidden] */
    const void* w3; int qt_3;
    int hidden;
    const void* gate_inp; int qt_gate_inp;             /* router [E, d] */
    const void* gate_exps; const void* up_exps; int qt_gu;   /* [E] x [ffn, d] */
    const void* down_exps; int qt_dn;                        /* [E] x [d, ffn] */
    int64_t stride_gu, stride_dn;                            /* bytes per expert */
    const void* gate_sh; const void* up_sh; int qt_sh_gu;    /* [shared, d] */
    const void* down_sh; int qt_sh_dn;                       /* [d, shared] */
    int shared_hidden;
} orc_mla_layer_w;

typedef struct {
    int dim, n_layers, n_heads, nope, rope, v_dim, dc, vocab, max_seq;
    int n_experts, top_k, expert_ffn;
    int nthreads;
    const void* wte; int qt_wte;
    const float* ln_f;
    const void* lm_head; int qt_lm;     /* NULL -> tied to wte */
    const orc_mla_layer_w* layers;
} orc_mla_cfg;

typedef struct orc_mla orc_mla;
orc_mla* orc_mla_create(const orc_mla_cfg* cfg);
void     orc_mla_destroy(orc_mla* m);
/* MLAInference::forward (infer/infer_mla.cpp:66-106) with
 * DeepseekMLAImpl::forward / forward_moe (deepseek_mla_layer.cu:171-350)
 * as intended at any start_pos: keys/values of positions < start_pos come
 * from the expanded per-layer cache (k_pe rotated, K_nope, V per head;
 * core/buffer.h:70-92 layout).  logits [T, vocab] or the last row. */
int      orc_mla_forward(orc_mla* m, const int* ids, int T, int start_pos, float* logits, int last_only);
int      orc_mla_generate(orc_mla* m, const int* prompt, int n_prompt, int steps, int* out_ids);
/* the expanded cache of one layer: k_pe [max_seq][rope], k_nope
 * [max_seq][H*nope], v [max_seq][H*v] (which: 0, 1, 2) */
const float* orc_mla_cache(orc_mla* m, int layer, int which);
/* Load cache positions 0..n_pos-1 of one layer from latent records
 * rec [n_pos][dc + rope] = [RMSNorm(c_kv)*k_norm | RoPE(k_pe)] (the GPU
 * engine's cache layout): k_pe copied, K_nope and V expanded through
 * W_kv_b exactly as orc_mla_forward stores its own rows. */
int orc_mla_load_latent(orc_mla* m, int layer, const float* rec, int n_pos);
/* Test hook: tap [n_layers][max_seq][dc + rope] receives the latent record
 * of every row orc_mla_forward stores (NULL: off). */
void orc_mla_set_latent_tap(orc_mla* m, float* tap);

/* ---- RINA Jamba hybrid (SSM + RINA-MLA layers, GQAInference) -------- */
enum { ORC_JAMBA_SSM = 0, ORC_JAMBA_RMLA = 1 };
typedef struct {
    int type;                           /* ORC_JAMBA_SSM or ORC_JAMBA_RMLA */
    int qt;                             /* quant type of every linear of the layer */
    const float* ln1; const float* ln2; /* LayerNorm weights [d] */
    const void* w_dq;                   /* SSM: path.w_dq [dc, d]; RMLA: path.w_dqkv [dc, d] */
    const float* q_norm;                /* [dc] */
    const void* w_mem[3];               /* SSM: [H*dh, dc] */
    const void* w_decay[3];             /* SSM: [H, dc] */
    const void* w_out;                  /* SSM: [d, d + H*dh] */
    const void* w_uq;                   /* RMLA: [H*dh, dc] */
    const void* w_uk;                   /* RMLA: [Hkv*dh, dc] */
    const void* w_k2v;                  /* RMLA: [Hkv*dh, Hkv*dh] */
    const void* w_qr;                   /* RMLA: [H*dhr, d] */
    const void* w_kr;                   /* RMLA: [Hkv*dhr, d] */
    const void* c_proj;                 /* RMLA: [d, H*dh] */
    const float* rope_q_cos; const float* rope_q_sin;   /* RMLA: [max_pos][dhr/2] */
    const float* rope_k_cos; const float* rope_k_sin;
    const void* w1; const void* w2; const void* w3;     /* SwiGLU [hidden, d], [d, hidden] */
} orc_jamba_layer_w;

typedef struct {
    int dim, n_layers, n_heads, n_kv_heads, head_dim, dhr, dc, ssm_steps, hidden, vocab, max_seq;
    int nthreads;
    const void* wte; int qt_wte;
    const float* ln_f;                  /* LayerNorm */
    const void* lm_head; int qt_lm;     /* NULL -> tied to wte */
    const orc_jamba_layer_w* layers;
    /* RINA-MLA cache form: ORC_KV_FP32, or ORC_KV_Q2K_Q1V (the key content
     * part packed as q2_1, the RoPE part kept fp32, values as q1_0;
     * rina/model_jamba_qw2.py:175-177); head_dim == 64 for the latter */
    int rmla_kv_mode;
} orc_jamba_cfg;

typedef struct orc_jamba orc_jamba;
orc_jamba* orc_jamba_create(const orc_jamba_cfg* cfg);
void       orc_jamba_destroy(orc_jamba* m);
/* GQAInference::forward (infer_gqa.cpp:75-105) over RinaSSMImpl
 * (arch/ssm/rina_ssm_layer.cu:90-126, kernels/ssm_kernels_fp32.cu:6-47)
 * and RinaMLAImpl (arch/mla/rina_mla_layer.cu:65-98) layers.  Those layers
 * keep no state, so the reference's semantics are a full recompute over
 * all tokens each step (tests/test_infer.cu:58-80).  This restatement
 * carries the scan state (log-cumsum, weighted cumsum) and the RINA-MLA
 * K/V rows across calls, in the same per-position fp32 operation order, so
 * a call at start_pos continuing the previous calls equals the full
 * recompute bit for bit; start_pos == 0 resets the state. */
int        orc_jamba_forward(orc_jamba* m, const int* ids, int T, int start_pos, float* logits, int last_only);
/* greedy decode: full prefill, then steps-1 incremental steps */
int        orc_jamba_generate(orc_jamba* m, const int* prompt, int n_prompt, int steps, int* out_ids);
/* greedy decode with the reference's full recompute at every step */
int        orc_jamba_generate_recompute(orc_jamba* m, const int* prompt, int n_prompt, int steps, int* out_ids);
/* packed RINA-MLA cache of layer l (rmla_kv_mode ORC_KV_Q2K_Q1V): part 0 the
 * key content q2_1 blocks [max_seq][Hkv][head_dim/32], 1 the value q1_0
 * records [max_seq][Hkv][head_dim/32]; NULL otherwise */
const uint8_t* orc_jamba_packed_cache(orc_jamba* m, int layer, int part);
/* fp32 rows of a RINA-MLA layer's cache as attention reads them: which 0
 * keys [max_seq][Hkv][head_dim + dhr], 1 values [max_seq][Hkv][head_dim]
 * (q2k_q1v mode: past rows hold their dequantized packs) */
const float* orc_jamba_fp32_cache(orc_jamba* m, int layer, int which);

int orc_num_threads(void);

#ifdef __cplusplus
}
#endif
#endif
