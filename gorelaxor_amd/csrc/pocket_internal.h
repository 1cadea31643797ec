// pocket_internal.h - the pocket-TTS driver's state, shared by its files
// (pocket_step.hip: the flow-LM transformer; pocket_flow.hip: the flow head).
#pragma once

#include <map>
#include <string>
#include <vector>

#include "grx_internal.h"

// A matrix of the flow head: Q8_0 (the float route of a weight that keeps
// its rows) or float32 [rows][cols]
struct FlowMat {
    int rows = 0, cols = 0;
    grx_weight *q8 = nullptr;
    float *f32 = nullptr;
};

struct FlowRes {
    FlowMat ada, fc1, fc2;
    float *norm_w = nullptr, *norm_b = nullptr, *ada_b = nullptr, *b1 = nullptr, *b2 = nullptr;
};

// SimpleMLPAdaLN of pockettts/lm.go:27-53 and its per-frame buffers
struct FlowHead {
    bool on = false, ready = false;
    int dim = 0, depth = 0, steps = 0;
    FlowMat cond, input, final_ada, out;
    float *cond_b = nullptr, *input_b = nullptr, *final_ada_b = nullptr, *out_b = nullptr;
    std::vector<FlowRes> res;
    float *tc = nullptr;      // [steps][dim] time conditions
    float *noise = nullptr;   // [max_pos][ldim] the caller's noise, one row a frame
    float *y = nullptr, *yi = nullptr, *sy = nullptr, *h = nullptr, *n = nullptr, *mm = nullptr, *mod = nullptr;
    float *cur = nullptr, *v = nullptr;
};

struct PLayer {
    grx_weight *qkv = nullptr, *out = nullptr, *ff1 = nullptr, *ff2 = nullptr;
    float *n1w, *n1b, *n2w, *n2b;
    float *k, *v;
};

struct grx_pocket {
    grx_ctx *ctx = nullptr;
    grx_pocket_hparams hp{};
    std::string sha;  // general.source.sha256 of the model file it was loaded from ("" when built from tensors)
    std::map<std::string, std::vector<uint8_t>> host;
    bool ready = false;
    std::vector<PLayer> L;
    std::vector<void *> allocs;
    float *input = nullptr, *bos = nullptr, *onw = nullptr, *onb = nullptr, *eosw = nullptr;
    float eosb = 0.f;
    float *rope_cos = nullptr, *rope_sin = nullptr;
    // activations, room for max_pos rows
    float *x = nullptr, *q = nullptr, *att = nullptr, *ff = nullptr;
    int8_t *att_q = nullptr, *ff_q = nullptr;
    float *att_s = nullptr, *ff_s = nullptr;
    float *lat = nullptr;                     // latents of a run of frames
    float *out_hist = nullptr, *eos_hist = nullptr;
    int *pos = nullptr, *frame = nullptr;
    int pos_host = 0;
    int lat_cap = 0;
    hipGraphExec_t exec = nullptr;
    hipGraph_t graph = nullptr;
    FlowHead flow;
    hipGraphExec_t speak_exec = nullptr;  // a frame and its flow head, captured
    hipGraph_t speak_graph = nullptr;
};

// pocket_step.hip
grx_status pocket_finalize(grx_pocket *m);
grx_status pocket_enqueue_frame(grx_pocket *m, hipStream_t st, const float *lat_base, const int *frame);
grx_status pocket_alloc(grx_pocket *m, size_t bytes, void **out);
// pocket_flow.hip
bool pocket_flow_tensor(const grx_pocket *m, const std::string &name, size_t *bytes_a, size_t *bytes_b);
grx_status pocket_flow_finalize(grx_pocket *m);
// the flow head's weights and its allocations from index mark of m->allocs on
void pocket_flow_release(grx_pocket *m, size_t mark);
grx_status pocket_flow_enqueue(grx_pocket *m, hipStream_t st);

