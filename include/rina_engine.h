/*
 * rina_engine.h — C-ABI of the host C++ engine (model config, weight map,
 * Inference orchestrators) built on rina_hip.h.  It is the binding surface
 * a caller without C++ (Python ctypes, the test harness, a cgo/JNI stub)
 * uses to drive the engine's Inference interface
 * (rina-engine/src/infer/infer_base.h:10-31) and the greedy decode loop of
 * rina-engine/src/main.cpp:666-690.  Device pointers unless stated;
 * `stream` is a hipStream_t.  Status returns follow rina_hip.h.
 */
#ifndef RINA_ENGINE_H
#define RINA_ENGINE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct rina_model rina_model;   /* ModelConfig + TensorMap */
typedef struct rina_infer rina_infer;   /* Inference */

/* Parse the model header JSON (keys of core/config.h:26-63 and
 * loader.cpp:43-84).  NULL on a parse error (see rina_engine_last_error). */
rina_model* rina_model_create(const char* config_json);
void rina_model_destroy(rina_model* m);

/* load_model (rina-engine/src/loader.cpp:149-152): a .rinn file, or a
 * directory holding weights.rinn (512-byte header, JSON config, tensor
 * index, data; tools/convert_llama_to_rinn.py:97-123 writes it).  Every
 * tensor is uploaded to device memory the model owns (freed by
 * rina_model_destroy).  FP32, Q4_0 and Q4_0F tensors, as the reference's
 * reader; NULL on a missing file, a bad magic, a truncated file or another
 * quant type (the reference prints and leaves that tensor empty), with the
 * reason in rina_engine_last_error and nothing left allocated. */
rina_model* rina_model_load(const char* path);

/* Register one tensor under its reference name (e.g.
 * "transformer.h.0.attn.w_q.weight").  data: device pointer to the packed
 * tensor in `quant_type` (core/quant.h ids); shape [ndim] with the row
 * count first.  The engine borrows the memory: the caller keeps it alive
 * for the model's lifetime (the role of WeightTensor::to_device,
 * core/tensor.h:18-27, when the caller owns the upload). */
int rina_model_add_tensor(rina_model* m, const char* name, int quant_type, int ndim, const int64_t* shape,
                          void* data);

/* create_inference(arch) + Inference::init.  arch: "gqa" (the reference
 * picks "mla" when layer 0's type contains "deepseek").  kv_mode overrides
 * the config's kv_quant_mode when not NULL ("fp32","q8","q4","q4k_q2v",
 * "q2","q2k_q1v"); max_seq > 0 overrides max_seq_len. */
rina_infer* rina_infer_create(rina_model* m, const char* arch, const char* kv_mode, int max_seq);
void rina_infer_destroy(rina_infer* inf);

/* Inference::forward: ids [B,T] (device), logits [B*T, vocab] (device). */
int rina_infer_forward(rina_infer* inf, const int* ids, float* logits, int B, int T, int start_pos, void* stream);

/* Greedy generation (host prompt in, host ids out): prefill + steps-1 decode
 * steps; use_graph replays the decode step as one HIP graph.  decode_ms
 * (host, may be NULL) receives the device time of the steps-1 decodes. */
int rina_infer_generate(rina_infer* inf, const int* prompt, int n_prompt, int steps, int* out_ids, int use_graph,
                        void* stream, float* decode_ms);

/* Continue the device greedy loop of the last rina_infer_generate for
 * `steps` more tokens (same stream rules); out_ids: host, steps ids. */
int rina_infer_decode(rina_infer* inf, int steps, int* out_ids, int use_graph, void* stream, float* decode_ms);

/* One layer's K (which_v=0) / V (1) cache region (device pointer, bytes). */
int rina_infer_kv_region(rina_infer* inf, int layer, int which_v, void** ptr, size_t* bytes);

/* Parity tap (test hook, no reference counterpart): device buffer
 * [n_layers][2][max_seq][kv_dim] fp32 that receives the K rows (as cached:
 * pre- or post-RoPE) and V rows appended by host-position
 * rina_infer_forward calls, so a caller can re-pack them and compare the
 * cache bytes.  NULL turns it off. */
int rina_infer_set_kv_tap(rina_infer* inf, float* tap);

/* Message of the last failure on this thread ("" if none). */
const char* rina_engine_last_error(void);

#ifdef __cplusplus
}
#endif
#endif
