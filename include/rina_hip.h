/*
 * rina_hip.h — C-ABI of the MI355X (gfx950) decode hot path of the RINA
 * engine (rina-engine).  Plain pointers and sizes; every pointer argument
 * is device memory unless stated; `stream` is a hipStream_t (NULL = the
 * null stream).  Every entry point is stream-ordered, never synchronizes,
 * and returns RINA_OK (0) or a negative status.
 *
 * Each declaration names the reference interface it replaces
 * (paths relative to the reference repository root).
 */
#ifndef RINA_HIP_H
#define RINA_HIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---------------------------------------------------- */
#define RINA_OK             0
#define RINA_ERR_ARG       -1   /* null pointer, negative or zero size     */
#define RINA_ERR_QTYPE     -2   /* quant type / KV format not supported    */
#define RINA_ERR_SHAPE     -3   /* K % 32 != 0 for Q4 types, K too large   */
#define RINA_ERR_RANGE     -4   /* position beyond the cache capacity      */
#define RINA_ERR_HIP       -5   /* HIP runtime error (launch, allocation)  */
#define RINA_ERR_WORKSPACE -6   /* caller workspace too small              */

/* ---- quant type ids: rina-engine/src/core/quant.h:9-14 --------------- */
#define RINA_QT_Q2_1      1
#define RINA_QT_Q1_0      2
#define RINA_QT_Q4_0      5
#define RINA_QT_FP32      6
#define RINA_QT_Q4_0F     7
#define RINA_QT_GGML_Q2_K 10

/* ---- KV cache modes: rina-engine/src/core/buffer.h:49 ---------------- */
#define RINA_KV_FP32     0
#define RINA_KV_Q8       1
#define RINA_KV_Q4       2
#define RINA_KV_Q4K_Q2V  3
#define RINA_KV_Q2       4
#define RINA_KV_Q2K_Q1V  5

/* ---- KV block formats (32 values per block) -------------------------- */
#define RINA_KVF_Q8_0  1   /* 34 B: fp16 scale + 32 x int8          */
#define RINA_KVF_Q4_0  2   /* 18 B: fp16 scale + 16 B nibbles (q+7) */
#define RINA_KVF_Q2_1  3   /* 10 B: fp16 amax + 8 B 2-bit (q+1)     */
#define RINA_KVF_Q1_0  4   /*  6 B: fp16 amax + u32 sign bits       */

/* ====================================================================== */
/* Quantized matvec                                                        */
/* ====================================================================== */

/* out[M,N] = in[M,K] . W[N,K]^T with W packed along K in `quant_type`
 * (RINA_QT_Q4_0, RINA_QT_Q4_0F, RINA_QT_GGML_Q2_K, RINA_QT_FP32).
 * Replaces launch_linear_dispatch (rina-engine/src/ops/linear.h:7-10,
 * ops/linear.cu:140-167): Q4_0 -> :60-95, Q4_0F -> :98-133, Q2_K -> the
 * fused M=1 kernel :406-442 / M>1 :445-483 (flat element indexing), FP32 ->
 * kernels/linear_fp32.cu:5-26.  Q4 types need K % 32 == 0.  input == output
 * is allowed and computed out of place through library scratch (the
 * reference's in-place calls race, arch/gqa/gqa_layer.cu:272). */
int rina_hip_linear(const void* weight, int quant_type, const float* input,
                    float* output, int M, int N, int K, void* stream);

/* Fused matvec launch (no single reference counterpart: it fuses calls the
 * reference makes back to back).  Up to 6 weight segments share one input
 * vector and one launch (M == 1 Q4_0 / Q4_0F / Q2_K rows of K <= 8192,
 * K % 32 == 0; other shapes run 3 segments per launch):
 *   RINA_EPI_STORE   out_s = W_s . x          (q/k/v: gqa_layer.cu:139-141)
 *   RINA_EPI_ADD     out_s = out_s + W_s . x  (w_o/w2 + launch_add:
 *                                              gqa_layer.cu:272-273,282-283)
 *   RINA_EPI_SWIGLU  out_0 = silu(W_0 . x) * (W2_0 . x)
 *                                             (w1, w3, launch_silu_mul:
 *                                              gqa_layer.cu:278-281)
 * All segments share quant_type and K.  input must not alias any output.
 * prologue normalizes each input row before the product, fusing the
 * norm launch that precedes these matvecs in the reference:
 *   RINA_PRO_NONE       x used as is
 *   RINA_PRO_RMSNORM    x * rsqrt(mean(x^2) + eps) * norm_w
 *                       (ops/rms_norm.cu:5-29, gqa_layer.cu:136,277)
 *   RINA_PRO_LAYERNORM  (x - mean) * rsqrt(var + eps) * norm_w
 *                       (kernels/pytorch_ln_kernel.cu:4-35) */
#define RINA_EPI_STORE  0
#define RINA_EPI_ADD    1
#define RINA_EPI_SWIGLU 2
#define RINA_PRO_NONE      0
#define RINA_PRO_RMSNORM   1
#define RINA_PRO_LAYERNORM 2
typedef struct {
    const void* weight;    /* [N, K] packed                              */
    const void* weight2;   /* RINA_EPI_SWIGLU: the up projection [N, K]  */
    float* out;            /* [M, N]                                     */
    int N;
} rina_linear_seg;
int rina_hip_linear_fused(const rina_linear_seg* segs, int nseg, int quant_type,
                          const float* input, int M, int K, int epilogue,
                          int prologue, const float* norm_w, float eps,
                          void* stream);

/* rina_hip_linear_fused that also stores the normalized input row
 * (prologue != RINA_PRO_NONE, M == 1) into norm_out [K]: the reference's
 * norm launch and the first matvec that reads it in one launch, with the
 * normalized row left for later consumers (the SSM layer's W_dq and W_out,
 * arch/ssm/rina_ssm_layer.cu:93-112).  norm_out must not alias input or
 * an output. */
int rina_hip_linear_fused_ex(const rina_linear_seg* segs, int nseg, int quant_type,
                             const float* input, int M, int K, int epilogue,
                             int prologue, const float* norm_w, float eps,
                             float* norm_out, void* stream);

/* ====================================================================== */
/* Weight formats                                                          */
/* ====================================================================== */

/* Pack n fp32 values (n % 32 == 0) into RINA_QT_Q4_0 (18 B blocks, fp16
 * RNE scale) or RINA_QT_Q4_0F (20 B blocks, fp32 scale).  Replaces
 * pack_q4_0 / pack_q4_0_f (rina-engine/tools/q4_pack.py:11-23,95-118):
 * scale = max(amax/7, 1e-10), q = sign(y)*min(floor(|y|+0.5),7). */
int rina_hip_pack_weights(int quant_type, const float* src, int64_t n,
                          void* dst, void* stream);

/* Pack n fp32 values (any n; ceil(n/32) blocks) into RINA_QT_Q4_0 with the
 * HF loader's rules (src/loader_hf.cpp:196-230): q = clamp(roundf(x/scale),
 * -7, 7), fp16 scale by truncation (exponent <= 0 -> 0, >= 31 -> 0x7FFF
 * class); a short last block leaves the missing elements' bytes zero. */
int rina_hip_pack_weights_hf(const float* src, int64_t n, void* dst, void* stream);

/* Dequantize n elements of a packed weight stream (flat element order) to
 * fp32.  Q2_K replaces dequant_block_q2_K_gpu (ops/linear.cu:322-338);
 * Q4_0/Q4_0F follow the matvec dequant rule (ops/linear.cu:77-81). */
int rina_hip_dequant_weights(int quant_type, const void* src, int64_t n,
                             float* dst, void* stream);

/* ====================================================================== */
/* KV cache                                                                */
/* ====================================================================== */

/* n % 32 == 0 values -> n/32 blocks of `kv_format`.  Replaces
 * launch_quantize_kv_to_q8_0 / launch_quantize_kv_to_q4_0 /
 * launch_quantize_k_fp32_to_q2_1 / launch_quantize_v_fp32_to_q1_0
 * (rina-engine/src/core/kernel_api.h:42-48; kernels/quantize.cu:74-270).
 * RINA_KVF_Q1_0 writes the documented 6-byte record [fp16][u32 LE]
 * (core/quant.h:44), not the 8-byte CUDA struct. */
int rina_hip_kv_quantize(int kv_format, const float* src, void* dst, int64_t n,
                         void* stream);

/* Inverse of rina_hip_kv_quantize.  Replaces launch_dequant_*
 * (core/kernel_api.h:44-49; kernels/quantize.cu:106-295). */
int rina_hip_kv_dequant(int kv_format, const void* src, float* dst, int64_t n,
                        void* stream);

/* Bytes of one layer's K (which_v = 0) or V (which_v = 1) cache region for
 * `mode` at max_seq positions of kv_dim values (buffer.cpp:104-132). */
size_t rina_hip_kv_region_bytes(int mode, int which_v, int max_seq, int kv_dim);

/* RoPE + quantize-on-append for one layer (gqa_layer.cu:147-190):
 *   q [T, H*dh] and k [T, Hkv*dh] are rotated in place with the NeoX pair
 *   rule of ops/rope.cu:125-149 (tables [pos, dh/2]; NULL = no rotation);
 *   K (pre-rotation when pre_rope) and V rows are written into the layer's
 *   cache regions at position pos0 = start_pos + (d_pos ? *d_pos : 0):
 *   mode 0: fp32 rows [max_seq, Hkv*dh]; mode 1..5: blocks of the mode's
 *   formats at block offset pos0*Hkv*dh/32. */
int rina_hip_rope_append(float* q, float* k, const float* v,
                         const float* rope_q_cos, const float* rope_q_sin,
                         const float* rope_k_cos, const float* rope_k_sin,
                         void* cache_k, void* cache_v, int mode, int pre_rope,
                         int T, int H, int Hkv, int dh, int start_pos,
                         const int* d_pos, int max_seq, void* stream);

/* Single-layer GQA attention for T query rows at positions
 * pos0..pos0+T-1 (pos0 = start_pos + (d_pos ? *d_pos : 0)).  Keys/values at
 * positions < pos0 are read from the layer's cache (fp32 or packed blocks,
 * dequantized in registers); positions >= pos0 from kcur/vcur [T, Hkv*dh]
 * fp32 (the current rows, post-RoPE).  Causal; query head h uses KV head
 * h / (H/Hkv); scale 1/sqrt(dh).  out [T, H*dh].
 * Replaces the composition of gqa_layer.cu:192-270 (cache dequant,
 * build_qkv_fp32.cu:8-33, flash_fp32.cu:12-111, row extraction).
 * pre_rope: cached keys are rotated with rope_k tables on read
 * (gqa_layer.cu:236-238).  `workspace` holds split-sequence partials;
 * rina_hip_gqa_attention_workspace() gives its size. */
size_t rina_hip_gqa_attention_workspace(int T, int H, int dh, int max_pos);
/* The position count up to which rina_hip_gqa_decode_attention over an fp32
 * cache with dh == 64 is one launch (1024; beyond it, or with a packed
 * cache, split + combine). */
int rina_hip_gqa_one_launch_positions(void);
int rina_hip_gqa_attention(const float* q, const float* kcur, const float* vcur,
                           const void* cache_k, const void* cache_v, int mode,
                           int pre_rope, const float* rope_k_cos,
                           const float* rope_k_sin, int T, int H, int Hkv, int dh,
                           int start_pos, const int* d_pos, int max_seq,
                           float* out, void* workspace, size_t workspace_bytes,
                           void* stream);

/* Decode step (T == 1, dh == 64) of one layer's attention with RoPE and the
 * cache append fused in: the result equals rina_hip_rope_append (pre_rope 0)
 * followed by rina_hip_gqa_attention, except that q and k are read raw and
 * left unmodified.  q [H*dh], k/v [Hkv*dh] are the current rows before RoPE;
 * K (rotated) and V are appended at pos0 = start_pos + (d_pos ? *d_pos : 0).
 * k_rot_out (optional, [Hkv*dh]) receives the rotated K row.  Same
 * workspace as rina_hip_gqa_attention.  Fuses gqa_layer.cu:147-270 for the
 * decode step (no counterpart as one reference call); RINA_ERR_SHAPE for
 * shapes it does not cover (the caller then uses the two-call form): q, k,
 * v, the RoPE tables and k_rot_out must be 16-byte aligned, fp32 caches
 * 16-byte aligned, packed caches 2-byte aligned. */
int rina_hip_gqa_decode_attention(const float* q, const float* k, const float* v,
                                  const float* rope_q_cos, const float* rope_q_sin,
                                  const float* rope_k_cos, const float* rope_k_sin,
                                  void* cache_k, void* cache_v, int mode, int H,
                                  int Hkv, int dh, int start_pos, const int* d_pos,
                                  int max_seq, float* out, float* k_rot_out,
                                  void* workspace, size_t workspace_bytes,
                                  void* stream);

/* rina_hip_gqa_decode_attention without a workspace argument, and it
 * allocates nothing: no counterpart in the reference; it is for callers
 * that cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  The chunk partials live in a
 * library-owned device array of rina_hip_noalloc_scratch_bytes() (1 MiB)
 * per device, held until the process ends; a call whose partials need more
 * (rina_hip_gqa_attention_workspace(1, H, 64, max_seq) bytes, e.g. more
 * than 62 query heads) returns RINA_ERR_WORKSPACE before launching.  All
 * calls on one device share that array: calls that overlap on one device
 * (different streams) race.  The first call on each device looks the array
 * up; make it outside graph capture.  The address is kept per device ordinal
 * for the life of the process: after hipDeviceReset it is stale, so this
 * entry point must not be called after a device reset in the same process
 * (nor rina_hip_argmax, whose key slot is kept the same way). */
size_t rina_hip_noalloc_scratch_bytes(void);
int rina_hip_gqa_decode_attention_noalloc(const float* q, const float* k, const float* v,
                                          const float* rope_q_cos, const float* rope_q_sin,
                                          const float* rope_k_cos, const float* rope_k_sin,
                                          void* cache_k, void* cache_v, int mode, int H,
                                          int Hkv, int dh, int start_pos, const int* d_pos,
                                          int max_seq, float* out, float* k_rot_out,
                                          void* stream);

/* ====================================================================== */
/* DeepSeek MLA (latent cache) and MoE                                     */
/* ====================================================================== */

/* Decode attention of one DeepseekMLAImpl layer at position
 * pos0 = start_pos + (d_pos ? *d_pos : 0), the intended math of
 * arch/mla/deepseek_mla_layer.cu:180-269 (the reference's start_pos > 0
 * branch is broken).  q [H*(nope+rope)] = W_q output ([H*nope | H*rope]);
 * kva [dc+rope] = W_kv_a output ([c_kv | k_pe]).  Appends the latent record
 * [RMSNorm(c_kv)*k_norm | RoPE(k_pe)] at pos0 of `cache` ([max_seq][dc+rope]
 * fp32) and writes out [H*v] = per head W_vb softmax-weighted latent, with
 * scores (q_nope.W_kb c + RoPE(q_rope).k_pe) / sqrt(nope+rope); W_kv_b
 * [H*(nope+v), dc] in flat element order (Q2_K, Q4_0, Q4_0F or fp32).
 * RoPE tables [max_seq][rope/2] (NULL: none).  dc % 64 == 0, dc <= 512,
 * dc + rope <= 640. */
size_t rina_hip_mla_attention_workspace(int H, int dc, int rope, int max_pos);
size_t rina_hip_mla_cache_bytes(int dc, int rope, int max_seq);
int rina_hip_mla_decode_attention(const float* q, const float* kva, const float* k_norm,
                                  float eps, const float* rope_cos, const float* rope_sin,
                                  const void* w_kv_b, int qt_kv_b, float* cache, int H,
                                  int nope, int rope, int v_dim, int dc, int start_pos,
                                  const int* d_pos, int max_seq, float* out,
                                  void* workspace, size_t workspace_bytes, void* stream);
/* The same with pos_hint: the largest position *d_pos can hold when the
 * launch runs (-1: max_seq - 1; ignored without d_pos).  It only selects the
 * kernels: below 256 positions, with dc == 512, rope <= 64, nope <= 128,
 * v <= 128 and Q2_K / Q4_0 / Q4_0F weights, one launch per call (every
 * workgroup of a head forms q_lat, the record and the softmax and computes
 * a quarter of W_vb), else the three-launch chunked path.  Either computes
 * every position correctly.  No counterpart in the reference: a graph that
 * is replayed at growing positions passes the bound of its replays. */
/* The position count below which rina_hip_mla_decode_attention_ex takes
 * the one-launch path (256). */
int rina_hip_mla_fused_positions(void);
int rina_hip_mla_decode_attention_ex(const float* q, const float* kva, const float* k_norm,
                                     float eps, const float* rope_cos, const float* rope_sin,
                                     const void* w_kv_b, int qt_kv_b, float* cache, int H,
                                     int nope, int rope, int v_dim, int dc, int start_pos,
                                     const int* d_pos, int max_seq, int pos_hint, float* out,
                                     void* workspace, size_t workspace_bytes, void* stream);

/* A prompt of T rows at positions 0..T-1 in one call: the prefill's causal
 * attention over all prompt rows (deepseek_mla_layer.cu:180-217, the
 * reference's expanded form: per head K = [W_kb c | RoPE(k_pe)],
 * V = W_vb c, scale 1/sqrt(nope + rope)).  q [T, H*(nope+rope)] and kva
 * [T, dc+rope] are the rows rina_hip_mla_decode_attention takes one at a
 * time; the T latent records are appended at positions 0..T-1 exactly as
 * T decode calls append them; out [T, H*v_dim].  dc <= 512,
 * nope + rope <= 256 and v_dim <= nope + rope (else RINA_ERR_SHAPE, before
 * any launch); w_kv_b Q2_K, Q4_0, Q4_0F or fp32.  The workspace (16-byte
 * aligned) holds rina_hip_mla_prompt_workspace() bytes of intermediate
 * rows. */
size_t rina_hip_mla_prompt_workspace(int T, int H, int nope, int rope, int v_dim, int dc);
int rina_hip_mla_prompt_attention(const float* q, const float* kva, const float* k_norm,
                                  float eps, const float* rope_cos, const float* rope_sin,
                                  const void* w_kv_b, int qt_kv_b, float* cache, int H,
                                  int nope, int rope, int v_dim, int dc, int T, int max_seq,
                                  float* out, void* workspace, size_t workspace_bytes, void* stream);

/* Router top-k of deepseek_mla_layer.cu:310-326 on the device: softmax of
 * the E logits, insertion top-k kept ascending (strict ">", the earlier
 * expert wins ties).  ids/probs [k] in that order.  E <= 256, k <= 16. */
int rina_hip_moe_topk(const float* logits, int n_experts, int k, int* ids,
                      float* probs, void* stream);

/* Routed experts of forward_moe (deepseek_mla_layer.cu:328-349) for one
 * token: for j < k (ascending): y_j = W_down[e_j] (SiLU(W_gate[e_j] x) *
 * (W_up[e_j] x)); h[i] += shared_out[i] + sum_j probs[j] y_j[i] (the sum
 * accumulated onto shared_out in j order, as the reference's saxpy chain).
 * Expert e's matrices start e*stride bytes into the stacked tensors of
 * n_experts experts; ids outside [0, n_experts) are skipped.  workspace: rina_hip_moe_workspace(k, ffn) bytes. */
size_t rina_hip_moe_workspace(int k, int ffn);
int rina_hip_moe_ffn(const float* x, const void* gate_exps, const void* up_exps,
                     const void* down_exps, int quant_type, int64_t stride_gate_up,
                     int64_t stride_down, int n_experts, const int* ids,
                     const float* probs, int k,
                     int d, int ffn, const float* shared_out, float* h, void* workspace,
                     size_t workspace_bytes, void* stream);

/* The MoE block over a prompt's T rows in one call (forward_moe,
 * deepseek_mla_layer.cu:291-350, for every row): h[T, d] += shared experts
 * + sum over each row's top-k of p_j * expert_j(RMSNorm(h_row, ln2)).  The
 * norm, the fp32 router logits and the shared experts run as T-row
 * products; the rows are then grouped by selected expert (the selection is
 * read back to the host once: the call synchronizes the stream) and each
 * expert runs as one product over its rows.  gate_sh / up_sh / down_sh may
 * be NULL with S == 0.  Any quant type rina_hip_linear_fused takes; the
 * workspace (16-byte aligned) holds rina_hip_moe_rows_workspace() bytes. */
size_t rina_hip_moe_rows_workspace(int T, int d, int n_experts, int k, int ffn, int shared_ffn);
int rina_hip_moe_rows(float* h, int T, const float* ln2, float eps, const void* gate_inp, int qt_inp,
                      const void* gate_sh, const void* up_sh, const void* down_sh, int shared_ffn, int qt_sh,
                      const void* gate_exps, const void* up_exps, const void* down_exps, int qt_exps,
                      int64_t stride_gu, int64_t stride_dn, int n_experts, int k, int d, int ffn,
                      void* workspace, size_t workspace_bytes, void* stream);

/* The whole MoE MLP block of one token (forward_moe,
 * deepseek_mla_layer.cu:291-350) for Q2_K experts and shared experts with an
 * fp32 router, in three launches and without the reference's host round
 * trip: a2 = RMSNorm(h, ln2); router logits = gate_inp a2; top-k of their
 * softmax (as rina_hip_moe_topk); G = SiLU(W_g a2) * (W_u a2) for the shared
 * FFN (shared_ffn rows) and the k selected experts (ffn rows each);
 * h += down_sh G_sh + sum_j probs[j] down[e_j] G_j, j ascending.  Shapes:
 * d, ffn <= 2048, d a multiple of 128, ffn, shared_ffn multiples of 32,
 * n_experts <= 64,
 * shared_ffn + k * ffn <= 16384; other shapes and formats return
 * RINA_ERR_SHAPE / RINA_ERR_QTYPE before anything is launched.  h, ln2,
 * gate_inp and workspace 16-byte aligned; workspace:
 * rina_hip_moe_block_workspace bytes (holds a2, the logits, the selected
 * ids / probs and G after the call). */
size_t rina_hip_moe_block_workspace(int d, int n_experts, int k, int ffn, int shared_ffn);
int rina_hip_moe_block(float* h, const float* ln2, float eps, const void* gate_inp, int qt_gate_inp,
                       const void* gate_sh, const void* up_sh, const void* down_sh, int shared_ffn,
                       const void* gate_exps, const void* up_exps, const void* down_exps, int quant_type,
                       int64_t stride_gate_up, int64_t stride_down, int n_experts, int k, int d, int ffn,
                       void* workspace, size_t workspace_bytes, void* stream);

/* ====================================================================== */
/* RINA Jamba hybrid (SSM and RINA-MLA layers)                             */
/* ====================================================================== */

/* One position of the InertiaWave SSM (arch/ssm/rina_ssm_layer.cu:98-109,
 * kernels/ssm_kernels_fp32.cu:6-47): dec_raw [steps][H] are the pre-sigmoid
 * decay projections, mem [steps][H*dh] the memory projections (steps <= 3,
 * missing steps act as decay 1, memory 0).  Per (h, d): da = d0 d1 d2,
 * ma = m0 d1 d2 + m1 d2 + m2, lcs += log(max(da, 1e-38)), ca = exp(lcs),
 * wcs += ma / max(ca, 1e-30), sf_out = ca wcs.  lcs / wcs [H*dh] carry the
 * scan across calls (reset != 0 starts it from zero), which reproduces the
 * reference's scan over the whole sequence. */
int rina_hip_ssm_step(const float* mem, const float* dec_raw, int steps, int H, int dh,
                      float* lcs, float* wcs, float* sf_out, int reset, void* stream);

/* T consecutive positions of rina_hip_ssm_step in one launch (a prompt's
 * scan; the reference's scan kernel walks the whole sequence,
 * kernels/ssm_kernels_fp32.cu:30-42): mem [steps][T][H*dh] and dec_raw
 * [steps][T][H] hold the projections of each position; the sf row of
 * position t goes to sf_out + t * sf_stride (sf_stride >= H*dh).  reset != 0
 * starts the scan from zero at the first position.  Every element advances
 * position by position with rina_hip_ssm_step's operations, so the rows and
 * the final state equal T one-position calls bit for bit. */
int rina_hip_ssm_scan(const float* mem, const float* dec_raw, int steps, int H, int dh, int T,
                      float* lcs, float* wcs, float* sf_out, int sf_stride, int reset, void* stream);

/* The SSM layer's step after cq = LN(W_dq x) in one launch: LN(cq, q_norm)
 * (LayerNorm, weight only, eps), mem_k = W_mem[k] . cq [H*dh] and
 * dec_k = W_decay[k] . cq [H] for k < steps, then rina_hip_ssm_step on them
 * (arch/ssm/rina_ssm_layer.cu:97-109: the q_norm launch, the 2*steps
 * projections and the scan, fused; no counterpart as one reference call).
 * w_mem / w_decay: arrays of `steps` packed weights [H*dh, dc] / [H, dc].
 * RINA_QT_Q4_0 / RINA_QT_Q4_0F only (else RINA_ERR_QTYPE), dc % 32 == 0 and
 * dc <= 256 (else RINA_ERR_SHAPE); both before anything is launched, so a
 * caller can fall back to rina_hip_linear_fused + rina_hip_ssm_step. */
int rina_hip_ssm_proj_step(const float* cq, const float* q_norm, float eps,
                           const void* const* w_mem, const void* const* w_decay,
                           int quant_type, int steps, int H, int dh, int dc,
                           float* lcs, float* wcs, float* sf_out, int reset, void* stream);

/* Decode attention of RinaMLAImpl (arch/mla/rina_mla_layer.cu:78-86) at
 * pos0 = start_pos + (d_pos ? *d_pos : 0): query [qa | RoPE_hf(qb)] per head
 * (qa [H*da], qb [H*db]), key [ka | RoPE_hf(kb)] and value v per KV head
 * (ka [Hkv*da], kb [Hkv*db], v [Hkv*dv]) appended at pos0 into fp32 caches
 * cache_k [max_seq][Hkv][da+db], cache_v [max_seq][Hkv][dv]; causal over
 * positions 0..pos0, head h uses KV head h / (H/Hkv), scale 1/sqrt(da+db);
 * out [H*dv].  HF RoPE pairs (2i, 2i+1) with tables [max_seq][db/2]
 * (ops/rope.cu:212-227; NULL: none).  dv == 64, 64 <= da + db <= 128,
 * contexts up to 2048 positions. */
size_t rina_hip_dq_attention_workspace(int H, int dq, int max_pos);
int rina_hip_dq_decode_attention(const float* qa, const float* qb, const float* ka,
                                 const float* kb, const float* v, const float* rope_q_cos,
                                 const float* rope_q_sin, const float* rope_k_cos,
                                 const float* rope_k_sin, float* cache_k, float* cache_v,
                                 int H, int Hkv, int da, int db, int dv, int start_pos,
                                 const int* d_pos, int max_seq, float* out, void* workspace,
                                 size_t workspace_bytes, void* stream);

/* A prompt's T rows at positions 0..T-1 of the RINA-MLA attention over the
 * fp32 caches in one call: every row's key [ka | HF-RoPE(kb)] and value
 * appended as rina_hip_dq_decode_attention appends them (bit for bit), then
 * one causal attention over the rows (rina_mla_layer.cu:78-86 over the
 * whole prompt; scale 1/sqrt(da + db)).  qa [T, H*da], qb [T, H*db],
 * ka [T, Hkv*da], kb [T, Hkv*db], v [T, Hkv*dv]; out [T, H*dv].
 * da + db <= 256 and dv <= da + db (else RINA_ERR_SHAPE, before any
 * launch); the workspace (16-byte aligned) holds
 * rina_hip_dq_prompt_workspace() bytes. */
size_t rina_hip_dq_prompt_workspace(int T, int H, int Hkv, int da, int db, int dv);
int rina_hip_dq_prompt_attention(const float* qa, const float* qb, const float* ka, const float* kb,
                                 const float* v, const float* rope_q_cos, const float* rope_q_sin,
                                 const float* rope_k_cos, const float* rope_k_sin, float* cache_k,
                                 float* cache_v, int H, int Hkv, int da, int db, int dv, int T,
                                 int max_seq, float* out, void* workspace, size_t workspace_bytes,
                                 void* stream);

/* rina_hip_dq_decode_attention with the cache form chosen by kv_mode:
 *   RINA_KV_FP32     cache_k [max_seq][Hkv][da+db] fp32, cache_v
 *                    [max_seq][Hkv][dv] fp32, cache_kr unused;
 *   RINA_KV_Q2K_Q1V  the q2 K / q1 V cache of the reference's RINA-MLA in
 *                    q2k_q1v mode (rina/model_jamba_qw2.py:175-177): cache_k
 *                    holds the key content part [max_seq][Hkv][da/32] as
 *                    q2_1 blocks, cache_kr the RoPE'd key part
 *                    [max_seq][Hkv][db] fp32 (training keeps it unquantized),
 *                    cache_v the values [max_seq][Hkv][dv/32] as 6-byte q1_0
 *                    records; da == 64, dv == 64.  The block codecs are
 *                    kernels/quantize.cu:74-185's (rina_hip_kv_quantize).
 * Positions before pos0 are read from the cache (dequantized), the current
 * position from the fp32 rows, which are then appended (packed), as the
 * GQA composition does (arch/gqa/gqa_layer.cu:192-270).
 * rina_hip_dq_kv_region_bytes gives each region's size: part 0 cache_k,
 * 1 cache_v, 2 cache_kr. */
size_t rina_hip_dq_kv_region_bytes(int kv_mode, int part, int max_seq, int Hkv, int da, int db, int dv);
int rina_hip_dq_decode_attention_kv(const float* qa, const float* qb, const float* ka,
                                    const float* kb, const float* v, const float* rope_q_cos,
                                    const float* rope_q_sin, const float* rope_k_cos,
                                    const float* rope_k_sin, int kv_mode, void* cache_k,
                                    void* cache_v, float* cache_kr, int H, int Hkv, int da,
                                    int db, int dv, int start_pos, const int* d_pos, int max_seq,
                                    float* out, void* workspace, size_t workspace_bytes,
                                    void* stream);

/* A prompt's T rows at positions start_pos .. start_pos + T - 1 of the
 * RINA-MLA attention in one call (the whole-sequence forward of
 * rina_mla_layer.cu:65-98), over the caches kv_mode selects as in
 * rina_hip_dq_decode_attention_kv (RINA_KV_FP32, or RINA_KV_Q2K_Q1V, the
 * cache of rina/model_jamba_qw2.py:175-177; else RINA_ERR_QTYPE): every
 * row's key and value are appended as rina_hip_dq_decode_attention_kv
 * appends them (the same bytes), then row t attends to the positions before
 * it through the cache and to its own position through its fp32 rows, as T
 * decode calls at those positions would (outputs equal within float
 * rounding).  qa [T, H*da], qb [T, H*db], ka [T, Hkv*da], kb [T, Hkv*db],
 * v [T, Hkv*dv]; out [T, H*dv].  dv == 64, 64 <= da + db <= 128, db even;
 * q2k_q1v: da == 64, caches 2-byte aligned; fp32: caches 4-byte aligned
 * (else RINA_ERR_SHAPE); start_pos + T <= max_seq (else RINA_ERR_RANGE).
 * No workspace. */
int rina_hip_dq_prompt_attention_kv(const float* qa, const float* qb, const float* ka,
                                    const float* kb, const float* v, const float* rope_q_cos,
                                    const float* rope_q_sin, const float* rope_k_cos,
                                    const float* rope_k_sin, int kv_mode, void* cache_k,
                                    void* cache_v, float* cache_kr, int H, int Hkv, int da,
                                    int db, int dv, int start_pos, int T, int max_seq, float* out,
                                    void* stream);

/* ====================================================================== */
/* Per-token glue                                                          */
/* ====================================================================== */

/* x[n,d] = x * rsqrt(mean(x^2) + eps) * w — launch_rms_norm_fp32
 * (ops/rms_norm.cu:5-34).  out may equal x. */
int rina_hip_rms_norm(const float* x, float* out, const float* w, int n, int d,
                      float eps, void* stream);
/* bias-free LayerNorm — launch_pytorch_ln_kernel
 * (kernels/pytorch_ln_kernel.cu:4-41).  out may equal x. */
int rina_hip_layer_norm(const float* x, float* out, const float* w, int n, int d,
                        float eps, void* stream);
/* RoPE on x [T, H, d]: hf_pairs = 0 -> pairs (i, i+d/2) (launch_rope_fp32,
 * ops/rope.cu:125-149); 1 -> pairs (2i, 2i+1) (launch_rope_fp32_hf,
 * ops/rope.cu:212-234).  Row t uses table row start_pos + (d_pos?*d_pos:0) + t. */
int rina_hip_rope(float* x, const float* cos_t, const float* sin_t, int T, int H,
                  int d, int start_pos, const int* d_pos, int hf_pairs,
                  void* stream);
/* out[n,d] = dequant(W[ids[i]]) for fp32 / Q4_0 / Q4_0F / Q2_K rows —
 * launch_embedding (ops/embedding.cu:200-230); ids are read at
 * ids + (d_pos ? *d_pos : 0).  vocab > 0: the table's row count; an id
 * outside [0, vocab) is clamped into it (the reference reads it unchecked,
 * which on a GPU faults); vocab <= 0: only negative ids are clamped (to 0)
 * and the caller guarantees id < rows. */
int rina_hip_embedding(const void* weight, int quant_type, const int* ids,
                       const int* d_pos, float* out, int n, int d, int vocab,
                       void* stream);
/* o = silu(g) * u — launch_silu_mul (ops/silu_mul.cu:5-12) */
int rina_hip_silu_mul(float* o, const float* g, const float* u, int64_t n, void* stream);
/* c = a + b — launch_add (ops/saxpy.cu:10-21) */
int rina_hip_add(float* c, const float* a, const float* b, int64_t n, void* stream);
/* d += p * s — launch_saxpy (ops/saxpy.cu:5-17) */
int rina_hip_saxpy(float* d, const float* s, float p, int64_t n, void* stream);
/* Greedy argmax with the strict ">" from -1e10 rule of sample()
 * (src/main.cpp:139-146): the lowest index wins ties (+0 and -0 are equal).
 * Writes the index to out_idx[0]; when d_pos is not NULL also stores it at
 * ids_out[*d_pos + 1] and increments *d_pos (device-side decode loop).
 * The candidates meet in one 8-byte key slot per device that the library
 * owns: calls that overlap on two streams of one device race on it (use
 * rina_hip_argmax_ws there).  The slot's address is kept per device ordinal
 * for the life of the process: not for use after hipDeviceReset. */
int rina_hip_argmax(const float* x, int n, int* out_idx, int* ids_out,
                    int* d_pos, void* stream);
/* rina_hip_argmax with the caller's key slot: key_slot is 8 bytes of
 * 8-byte-aligned device memory that holds zero before the first call (the
 * call leaves it zero again).  Calls with different slots never share
 * state, so decode loops on different streams can run together.  No
 * counterpart in the reference (its sample() runs on the host). */
int rina_hip_argmax_ws(const float* x, int n, int* out_idx, int* ids_out,
                       int* d_pos, void* key_slot, void* stream);

/* The greedy decode step's tail in fewer launches (no counterpart in the
 * reference, whose sample() runs on the host, main.cpp:139-146, and whose
 * next step starts with the embedding launch, ops/embedding.cu:6-230).
 *
 * rina_hip_linear_argmax: the fp32 LM head (rina_hip_linear_fused with one
 * segment, M = 1, the store epilogue and the optional norm prologue; the
 * same logits) that also writes the largest argmax key of the rows each of
 * its workgroups stored into keys[0 .. *nkeys) (8-byte aligned device
 * memory of max_keys keys; RINA_ERR_WORKSPACE when the launch needs more:
 * at most 8 per compute unit).  Keys are 64-bit: the order-preserving bits
 * of the value, then the complemented index (strict ">" from -1e10, the
 * lowest index among equal values, -0 as +0).  Other quant types return
 * RINA_ERR_QTYPE.
 *
 * rina_hip_argmax_partial: the first half of rina_hip_argmax_ws, merging
 * x's candidates into key_slot (which must hold zero).
 *
 * rina_hip_argmax_embed: the winner of keys[0 .. nkeys) (cleared again when
 * reset, as a key slot must be), then what rina_hip_argmax_ws does with it
 * (out_idx, ids_out[*d_pos + 1], *d_pos + 1; each optional), then row id of
 * the embedding table emb (quant type emb_qt, rows of d values, vocab rows;
 * ids outside it clamped) into h[0 .. d): the next decode step's input,
 * so that step needs no embedding launch. */
int rina_hip_linear_argmax(const rina_linear_seg* seg, int quant_type, const float* input, int K,
                           int prologue, const float* norm_weight, float eps, void* keys,
                           int max_keys, int* nkeys, void* stream);
int rina_hip_argmax_partial(const float* x, int n, void* key_slot, void* stream);
int rina_hip_argmax_embed(void* keys, int nkeys, int reset, int* out_idx, int* ids_out, int* d_pos,
                          const void* emb, int emb_qt, float* h, int d, int vocab, void* stream);

/* Measurement helper, no counterpart in the reference: one launch of
 * `grid` 256-thread workgroups that stream-reads bytes (rounded down to
 * 16) of src (16-byte aligned) and writes grid floats to sink.  Its time
 * is the plain-read ceiling the benchmark sets next to each matvec of the
 * same byte count. */
int rina_hip_read_probe(const void* src, int64_t bytes, int grid, float* sink, void* stream);

/* Library version / self-description. */
const char* rina_hip_version(void);

#ifdef __cplusplus
}
#endif
#endif
