// gguf_moe kernels: one position, or a batch of positions along the launch's y dimension.
#pragma once

#include <hip/hip_runtime.h>

#include "chunk.h"

namespace rq {

// A routed expert bank or a single (shared) expert, as the MoE kernels read it.
struct MoeBank {
    Planes P;          // planes of expert 0, row 0
    int64_t rows;      // rows per expert
};

struct MoeDims {
    int d_model, experts, top, hidden, hidden_shared;  // hidden_shared = 0: no shared expert
    int scoring, renormalize;
    int shared_gated;  // 1: the shared expert is weighted by shared_gate_act(gate . x); 0: by one
    float scale;
    int activation;       // act(gate x) * up x of every expert (act.h codes)
    int shared_gate_act;  // the shared gate's activation
    float act_factor;     // Scale's constant / PReLU's slope
    const float* sel_bias = nullptr;  // experts fp32: the top-k selection key is probability + bias
};

// Workspace carve-up (floats unless noted), all in one device buffer.
struct MoeWorkspace {
    float* logits;  // experts + 1 (router scores, then the shared gate score)
    int* ids;       // top (selected experts in ascending id)
    float* weights; // top + 1 (routing weights, then the shared expert's gate)
    float* h;       // top * hidden + hidden_shared (SiLU(gate) * up per slot)
};

size_t moe_workspace_bytes(const MoeDims& d);
MoeWorkspace moe_workspace(void* base, const MoeDims& d);

// Positions of a batch: launch dimension y picks position p, whose activations
// start p * x_stride bytes after x, workspace p * ws_stride bytes after the
// first position's, output p * y_stride floats after y and routing plane
// p * route_stride floats after route_dense.
struct MoeBatch {
    int64_t x_stride = 0, ws_stride = 0, y_stride = 0, route_stride = 0;
    int m = 1;
};

// Routes the position (ws.ids, ws.weights and route_dense when not null,
// topk_forward_body semantics, amd-nv-cpu.ll:4653-4716) and computes
// h[slot][f] = act(gate_slot[f] . x) * (up_slot[f] . x) for every routed slot
// and the shared expert.
hipError_t launch_moe_glu(int fmt, int xtype, const MoeDims& d, const MoeBank& gate, const MoeBank& up,
                          const MoeBank& gate_sh, const MoeBank& up_sh, const void* x, MoeWorkspace ws,
                          float* route_dense, const MoeBatch& b, int cus, hipStream_t stream);

// y[n] = sum_slot w_slot * (down_slot[n] . h_slot), routed slots in ascending expert id, then the shared expert.
hipError_t launch_moe_down(int fmt, const MoeDims& d, const MoeBank& down, const MoeBank& down_sh, MoeWorkspace ws,
                           float* y, const MoeBatch& b, int cus, hipStream_t stream);

}  // namespace rq
