// Device-side greedy decode loop shared by the Inference orchestrators
// (the loop of rina-engine/src/main.cpp:666-690, moved onto the GPU): the
// argmax kernel writes the next id into the device id buffer and advances a
// device position, so one decode step is position-independent and is
// captured once as a HIP graph and replayed.  An orchestrator whose kernels
// differ below and above some position (graph_split()) gets one graph per
// side, each captured with the bound of the positions it replays at.
// A decode step's tail is fused: the step's last launch (argmax + embedding)
// also writes the next step's embedding row into h, so a step is layers ->
// LM head -> argmax_embed (with an fp32 LM head the argmax's per-workgroup
// keys come out of the LM head launch itself); decode_more() embeds the
// first step's id once before its loop.
#pragma once
#include <hip/hip_runtime_api.h>
#include <string>
#include "infer/infer_base.h"
#include "rina_hip.h"

struct DeviceGreedyInference : Inference {
    int* d_ids = nullptr;      // [max_seq + 1]
    int* d_pos = nullptr;      // device position of the last id; d_pos[2..3]: this loop's argmax key slot
    int max_seq = 0;
    int vocab = 0;
    int gen_len = 0;           // ids valid in d_ids after the last generate / decode_more
    hipGraphExec_t graph[2] = {nullptr, nullptr};   // positions below / from graph_split()
    hipStream_t graph_stream[2] = {nullptr, nullptr};
    int pos_hint = -1;         // largest position of the next device-position run (-1: unknown)
    int h_pos = 0;             // host source of the first position's copy: outlives any queued copy
    std::string tag = "infer";
    static constexpr int kMaxKeys = 8192;   // argmax keys of a fused LM head: one per workgroup (<= 8 per CU)
    unsigned long long* d_keys = nullptr;
    int n_keys = 0;            // keys the last fused LM head wrote (0: the LM head was not fused)
    bool fuse_tail = false;    // set while a decode step is issued: run() skips the embedding and may fuse the argmax

    ~DeviceGreedyInference() override {
        for (auto& g : graph)
            if (g) (void)hipGraphExecDestroy(g);
        if (d_ids) (void)hipFree(d_ids);
        if (d_pos) (void)hipFree(d_pos);
        if (d_keys) (void)hipFree(d_keys);
    }

    // embedding -> layers -> final norm -> LM head for T ids at start_pos
    // (pos_dev: device position instead, T == 1); logits of the last row
    // only when last_only.
    virtual int run(const int* ids, const int* pos_dev, int T, int start_pos, float* logits, bool last_only,
                    hipStream_t s) = 0;
    // grow the activation buffers to n rows (caches are kept)
    virtual int ensure_cap(int n) = 0;
    // last-row logits buffer of the device loop
    virtual float* lm_buffer() = 0;
    // first position of the second decode graph (0: one graph for all)
    virtual int graph_split() const { return 0; }
    // the embedding table, the activation row h and its width, for the fused tail
    virtual const WeightTensor* emb_table() const = 0;
    virtual float* h_buffer() = 0;
    virtual int model_dim() const = 0;

    bool alloc_ids() {
        return hipMalloc(&d_ids, sizeof(int) * (max_seq + 1)) == hipSuccess &&
               hipMalloc(&d_pos, 4 * sizeof(int)) == hipSuccess && hipMemset(d_pos, 0, 4 * sizeof(int)) == hipSuccess &&
               hipMalloc(&d_keys, sizeof(unsigned long long) * kMaxKeys) == hipSuccess;
    }
    // LM head of a decode step with the argmax keys fused in, where the
    // head is fp32 (otherwise the plain launch; n_keys stays 0)
    int head_launch(const rina_linear_seg& seg, int qt, const float* x, int K, int pro, const float* nw, hipStream_t s) {
        if (fuse_tail && qt == RINA_QT_FP32)
            return rina_hip_linear_argmax(&seg, qt, x, K, pro, nw, 1e-5f, d_keys, kMaxKeys, &n_keys, s);
        return rina_hip_linear_fused(&seg, 1, qt, x, 1, K, RINA_EPI_STORE, pro, nw, 1e-5f, s);
    }
    // argmax of the step's logits and the next step's embedding row, one
    // launch after the fused LM head, two after a plain one
    int argmax_embed(hipStream_t s) {
        const WeightTensor* e = emb_table();
        if (n_keys > 0)
            return rina_hip_argmax_embed(d_keys, n_keys, 0, nullptr, d_ids, d_pos, e->data, (int)e->quant_type,
                                         h_buffer(), model_dim(), vocab, s);
        int rc = rina_hip_argmax_partial(lm_buffer(), vocab, d_pos + 2, s);
        if (rc) return rc;
        return rina_hip_argmax_embed(d_pos + 2, 1, 1, nullptr, d_ids, d_pos, e->data, (int)e->quant_type, h_buffer(),
                                     model_dim(), vocab, s);
    }
    // argmax with this inference's own key slot: two inferences decoding on
    // different streams never share it
    int argmax(hipStream_t s) { return rina_hip_argmax_ws(lm_buffer(), vocab, nullptr, d_ids, d_pos, d_pos + 2, s); }

    // A captured graph holds the activation pointers of its capture: every
    // ensure_cap() that re-allocates them must drop the graphs, so the next
    // decode_more() captures again on the new buffers.
    void drop_graphs() {
        for (int c = 0; c < 2; c++) {
            if (graph[c]) (void)hipGraphExecDestroy(graph[c]);
            graph[c] = nullptr;
            graph_stream[c] = nullptr;
        }
    }

    // (re)capture decode graph c, valid for device positions <= hint
    int capture(int c, int hint, hipStream_t s) {
        if (graph[c] && graph_stream[c] == s) return RINA_OK;
        if (graph[c]) { (void)hipGraphExecDestroy(graph[c]); graph[c] = nullptr; }
        hipGraph_t g = nullptr;
        pos_hint = hint;
        if (hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal) != hipSuccess) return RINA_ERR_HIP;
        int crc = decode_step(s);
        hipError_t ce = hipStreamEndCapture(s, &g);
        pos_hint = -1;
        if (crc) { if (g) (void)hipGraphDestroy(g); return crc; }
        if (ce != hipSuccess) return RINA_ERR_HIP;
        hipError_t ie = hipGraphInstantiate(&graph[c], g, nullptr, nullptr, 0);
        (void)hipGraphDestroy(g);
        if (ie != hipSuccess) { graph[c] = nullptr; return RINA_ERR_HIP; }
        graph_stream[c] = s;
        return RINA_OK;
    }

    // one decode step: h holds the step's embedding row (written by the
    // previous step's tail, or by decode_more() before its first step)
    int decode_step(hipStream_t s) {
        fuse_tail = true;
        n_keys = 0;
        int rc = run(d_ids, d_pos, 1, 0, lm_buffer(), true, s);
        fuse_tail = false;
        if (rc) return rc;
        return argmax_embed(s);
    }

    int generate(const int* prompt, int n, int steps, int* out, bool use_graph, hipStream_t s,
                 float* decode_ms) override {
        if (n < 1 || steps < 1 || n + steps - 1 > max_seq) { err_ = tag + ": prompt + steps exceed max_seq"; return RINA_ERR_RANGE; }
        for (int i = 0; i < n; i++)
            if (prompt[i] < 0 || prompt[i] >= vocab) {
                err_ = tag + ": prompt id " + std::to_string(prompt[i]) + " outside the vocabulary";
                return RINA_ERR_ARG;
            }
        int rc = ensure_cap(n);
        if (rc) return rc;
        // the caller's prompt is a host source of queued copies: every return
        // below waits for the stream first, so no copy outlives it
        auto drain = [&](int r) { (void)hipStreamSynchronize(s); return r; };
        if (hipMemcpyAsync(d_ids, prompt, sizeof(int) * n, hipMemcpyHostToDevice, s) != hipSuccess)
            return drain(RINA_ERR_HIP);
        h_pos = n - 1;
        if (hipMemcpyAsync(d_pos, &h_pos, sizeof(int), hipMemcpyHostToDevice, s) != hipSuccess)
            return drain(RINA_ERR_HIP);
        if ((rc = run(d_ids, nullptr, n, 0, lm_buffer(), true, s))) return drain(rc);
        if ((rc = argmax(s))) return drain(rc);
        if (hipStreamSynchronize(s) != hipSuccess) return RINA_ERR_HIP;
        gen_len = n + 1;
        if (hipMemcpyAsync(out, d_ids + n, sizeof(int), hipMemcpyDeviceToHost, s) != hipSuccess)
            return drain(RINA_ERR_HIP);
        if (steps == 1) {
            if (decode_ms) *decode_ms = 0.f;
            return hipStreamSynchronize(s) == hipSuccess ? RINA_OK : RINA_ERR_HIP;
        }
        return decode_more(steps - 1, out + 1, use_graph, s, decode_ms);
    }

    int decode_more(int steps, int* out, bool use_graph, hipStream_t s, float* decode_ms) override {
        if (gen_len < 1) { err_ = tag + ": decode_more before generate"; return RINA_ERR_ARG; }
        if (steps < 1 || gen_len + steps - 1 > max_seq) { err_ = tag + ": decode exceeds max_seq"; return RINA_ERR_RANGE; }
        const int split = graph_split();
        const int pos_first = gen_len - 1;   // position of the first step's id
        int rc = RINA_OK;
        if (use_graph) {
            // capture the graphs this call replays before the timed loop
            for (int c = 0; c < 2; c++) {
                const bool needed = c == 0 ? (split <= 0 || pos_first < split)
                                           : (split > 0 && pos_first + steps - 1 >= split);
                if (needed && (rc = capture(c, c == 0 && split > 0 ? split - 1 : -1, s))) return rc;
            }
        }
        hipEvent_t e0 = nullptr, e1 = nullptr;
        (void)hipEventCreate(&e0);
        (void)hipEventCreate(&e1);
        (void)hipEventRecord(e0, s);
        // the first step's embedding row (every later one comes from the
        // step before it)
        {
            const WeightTensor* e = emb_table();
            rc = rina_hip_embedding(e->data, (int)e->quant_type, d_ids, d_pos, h_buffer(), 1, model_dim(), vocab, s);
        }
        for (int i = 0; i < steps && rc == RINA_OK; i++) {
            const int pos = pos_first + i;
            if (use_graph) {
                const int c = split > 0 && pos >= split ? 1 : 0;
                rc = hipGraphLaunch(graph[c], s) == hipSuccess ? RINA_OK : RINA_ERR_HIP;
            } else {
                pos_hint = pos;
                rc = decode_step(s);
            }
        }
        (void)hipEventRecord(e1, s);
        if (rc == RINA_OK && hipMemcpyAsync(out, d_ids + gen_len, sizeof(int) * steps, hipMemcpyDeviceToHost, s) != hipSuccess)
            rc = RINA_ERR_HIP;
        if (hipStreamSynchronize(s) != hipSuccess && rc == RINA_OK) rc = RINA_ERR_HIP;
        float ms = 0.f;
        if (rc == RINA_OK) {
            gen_len += steps;
            (void)hipEventElapsedTime(&ms, e0, e1);
        }
        if (decode_ms) *decode_ms = ms;
        (void)hipEventDestroy(e0);
        (void)hipEventDestroy(e1);
        return rc;
    }
};
