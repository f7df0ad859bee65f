// Inference interface and name registry (rina-engine/src/infer/infer_base.h:10-31),
// with the HIP stream type.  forward() keeps the reference contract: ids
// [B,T] and logits [B,T,V] are device pointers, start_pos is the cache
// position of the first row (0 = prefill).  The greedy generation loop of
// main.cpp:666-690 is an added member that runs on the device.
#pragma once
#include <hip/hip_runtime_api.h>
#include <string>
#include "core/config.h"
#include "core/tensor.h"

struct Inference {
    virtual ~Inference() = default;
    virtual bool init(ModelConfig& cfg, const TensorMap& weights) = 0;
    // returns RINA_OK or a negative status (the reference's is void)
    virtual int forward(const int* ids, float* logits, int B, int T, int start_pos, hipStream_t stream) = 0;

    // Greedy decode of main.cpp:666-690: one prefill over the prompt, then
    // steps-1 single-token steps; ids of the steps generated tokens go to
    // out (host).  Decode steps run as one replayed HIP graph when
    // use_graph; decode_ms (optional) receives the device time of the
    // decode steps.
    virtual int generate(const int* prompt, int n_prompt, int steps, int* out, bool use_graph, hipStream_t stream,
                         float* decode_ms) = 0;
    // Continue the device decode loop of the last generate() for `steps`
    // more tokens (out: host, steps ids).
    virtual int decode_more(int steps, int* out, bool use_graph, hipStream_t stream, float* decode_ms) = 0;
    // Device pointer / size of one layer's K or V cache region.
    virtual int kv_region(int layer, int which_v, void** ptr, size_t* bytes) = 0;
    // Parity tap: device buffer [n_layers][2][max_seq][kv_dim] that receives
    // the fp32 K/V rows appended by host-position forward() calls (NULL: off).
    virtual int set_kv_tap(float* tap) = 0;
    virtual std::string last_error() const { return err_; }

protected:
    std::string err_;
};

using InferenceFactory = Inference* (*)();
void register_inference(const std::string& name, InferenceFactory factory);
Inference* create_inference(const std::string& name);
void register_all_inferences();
