// Inference interface and name registry (rina-engine/src/infer/infer_base.h:10-31),
// with the HIP stream type.  init() and forward() keep the reference's
// signatures: ids [B,T] and logits [B,T,V] are device pointers, start_pos is
// the cache position of the first row (0 = prefill), and forward() returns
// void.  A forward() that fails leaves its status in last_status() (RINA_OK
// or a negative RINA_ERR_*) and the reason in last_error(); run_forward()
// returns that status in one call.  The greedy generation loop of
// main.cpp:666-690, the cache accessors and the parity tap are added
// members.
#pragma once
#include <hip/hip_runtime_api.h>
#include <string>
#include "core/config.h"
#include "core/tensor.h"

struct Inference {
    virtual ~Inference() = default;

    // Initialize: allocate all buffers, build the layer pipeline
    virtual bool init(ModelConfig& cfg, const TensorMap& weights) = 0;

    // Run the model on one batch (reference contract, status in last_status())
    virtual void forward(const int* ids, float* logits, int B, int T, int start_pos, hipStream_t stream) = 0;

    // ---- added to the reference interface ----

    // forward(), then its status
    int run_forward(const int* ids, float* logits, int B, int T, int start_pos, hipStream_t stream) {
        status_ = 0;
        forward(ids, logits, B, T, start_pos, stream);
        return status_;
    }
    int last_status() const { return status_; }
    virtual std::string last_error() const { return err_; }

    // Greedy decode of main.cpp:666-690: one prefill over the prompt, then
    // steps-1 single-token steps; ids of the steps generated tokens go to
    // out (host).  Decode steps run as one replayed HIP graph when
    // use_graph; decode_ms (optional) receives the device time of the
    // decode steps.  These members have defaults, so an Inference written
    // against the reference's interface (init + forward only) still
    // compiles; the defaults report RINA_ERR_ARG.
    virtual int generate(const int* prompt, int n_prompt, int steps, int* out, bool use_graph, hipStream_t stream,
                         float* decode_ms) {
        (void)prompt; (void)n_prompt; (void)steps; (void)out; (void)use_graph; (void)stream; (void)decode_ms;
        return unsupported("generate");
    }
    // Continue the device decode loop of the last generate() for `steps`
    // more tokens (out: host, steps ids).
    virtual int decode_more(int steps, int* out, bool use_graph, hipStream_t stream, float* decode_ms) {
        (void)steps; (void)out; (void)use_graph; (void)stream; (void)decode_ms;
        return unsupported("decode_more");
    }
    // Device pointer / size of one layer's K or V cache region.
    virtual int kv_region(int layer, int which_v, void** ptr, size_t* bytes) {
        (void)layer; (void)which_v; (void)ptr; (void)bytes;
        return unsupported("kv_region");
    }
    // Parity tap: device buffer [n_layers][2][max_seq][kv_dim] that receives
    // the fp32 K/V rows appended by host-position forward() calls (NULL: off).
    virtual int set_kv_tap(float* tap) {
        (void)tap;
        return unsupported("set_kv_tap");
    }

protected:
    std::string err_;
    int status_ = 0;
    int unsupported(const char* what) {
        err_ = std::string(what) + ": not provided by this Inference";
        return -1;   // RINA_ERR_ARG
    }
    // record a failure of forward(): status and reason
    void set_status(int rc, const std::string& why = std::string()) {
        status_ = rc;
        if (rc && !why.empty()) err_ = why;
    }
};

using InferenceFactory = Inference* (*)();
void register_inference(const std::string& name, InferenceFactory factory);
Inference* create_inference(const std::string& name);
void register_all_inferences();
