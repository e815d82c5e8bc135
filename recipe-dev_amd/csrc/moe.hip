// gguf_moe decode step (one position) on gfx950.
//
// Reference: lower_gguf_moe (recipe.rs:23415-23459) emits router Contraction ->
// TopK -> ExpertIn(gate), ExpertIn(up) -> silu(gate)*up -> ExpertOut(down), and a
// shared expert as a one-expert bank weighted by its gate; the device bodies
// are topk_forward_wave_body (amd-nv-cpu.ll:4489-4652) and packed_lanes_body
// modes 1/2 (amd-nv-cpu.ll:2897-2986, 3041-3086).
//
// Here the router runs as an F16 matvec, then:
//   moe_topk  one wave: repeated wave argmax (the lower expert on a tie), the
//             routing weights, slots in ascending expert id;
//   moe_glu   one lane group per (slot, hidden row): the gate and up rows of the
//             slot's expert are read together against x staged in LDS, and
//             silu(gate) * up is written per slot (routed slots, then shared);
//   moe_down  one lane group per output row: its lanes walk the chunks of every
//             slot's down row (K = all slots' hidden widths back to back, h staged
//             in LDS), scale each chunk by its slot's weight, and reduce across
//             lanes; no atomics, no second pass.
#include "moe.h"
#include "stage.h"

namespace rq {

static size_t al(size_t v) { return (v + 255) & ~size_t(255); }

size_t moe_workspace_bytes(const MoeDims& d) {
    return al(sizeof(float) * (size_t)(d.experts + 1)) + al(sizeof(int) * (size_t)d.top) +
           al(sizeof(float) * (size_t)(d.top + 1)) + al(sizeof(float) * ((size_t)d.top * d.hidden + d.hidden_shared));
}

MoeWorkspace moe_workspace(void* base, const MoeDims& d) {
    char* p = static_cast<char*>(base);
    MoeWorkspace w;
    w.logits = reinterpret_cast<float*>(p);
    p += al(sizeof(float) * (size_t)(d.experts + 1));
    w.ids = reinterpret_cast<int*>(p);
    p += al(sizeof(int) * (size_t)d.top);
    w.weights = reinterpret_cast<float*>(p);
    p += al(sizeof(float) * (size_t)(d.top + 1));
    w.h = reinterpret_cast<float*>(p);
    return w;
}

__device__ __forceinline__ float sigmoidf_dev(float v) { return 1.0f / (1.0f + expf(-v)); }

// (value, index) argmax across the wave; a higher value wins, the lower index on a tie.
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(v, off);
        const int oi = __shfl_xor(i, off);
        const bool take = (oi >= 0) && (i < 0 || ov > v || (ov == v && oi < i));
        if (take) {
            v = ov;
            i = oi;
        }
    }
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

// Experts per lane: E <= 64 * kTopkSlots.
constexpr int kTopkSlots = 32;

__global__ void __launch_bounds__(64) moe_topk_kernel(MoeDims d, MoeWorkspace ws, float* route_dense) {
    __shared__ int pick_id[64];
    __shared__ float pick_val[64];
    const int lane = threadIdx.x;
    const int E = d.experts;
    uint32_t taken = 0;  // bit i: expert lane + 64 i already picked
    for (int p = 0; p < d.top; ++p) {
        float bv = 0.f;
        int bi = -1;
        for (int i = 0; i < kTopkSlots; ++i) {
            const int e = lane + 64 * i;
            if (e >= E) break;
            if (taken & (1u << i)) continue;
            const float v = ws.logits[e];
            if (bi < 0 || v > bv) {  // ascending e: keeps the lower expert on a tie
                bv = v;
                bi = e;
            }
        }
        wave_argmax(bv, bi);
        if (bi >= 0 && (bi & 63) == lane) taken |= 1u << (bi >> 6);
        if (lane == 0) {
            pick_id[p] = bi;
            pick_val[p] = bv;
        }
    }
    __syncthreads();
    const bool sigmoid = d.scoring != 0, renorm = d.renormalize != 0;
    // Maximum and total over the kept experts (renormalized) or over all.
    float maximum, total;
    if (renorm) {
        maximum = pick_val[0];
        float t = 0.f;
        for (int p = lane; p < d.top; p += 64) t += sigmoid ? sigmoidf_dev(pick_val[p]) : expf(pick_val[p] - maximum);
        total = wave_sum(t);
    } else {
        float mx = -INFINITY;
        for (int e = lane; e < E; e += 64) mx = fmaxf(mx, ws.logits[e]);
        maximum = wave_max(mx);
        float t = 0.f;
        for (int e = lane; e < E; e += 64) t += sigmoid ? sigmoidf_dev(ws.logits[e]) : expf(ws.logits[e] - maximum);
        total = wave_sum(t);
    }
    const float denom = (renorm || !sigmoid) ? total : 1.0f;
    if (route_dense)
        for (int e = lane; e < E; e += 64) route_dense[e] = 0.f;
    __syncthreads();
    for (int p = lane; p < d.top; p += 64) {
        const int id = pick_id[p];
        int slot = 0;  // rank of this expert among the picked ids
        for (int q = 0; q < d.top; ++q) slot += pick_id[q] < id;
        const float raw = sigmoid ? sigmoidf_dev(pick_val[p]) : expf(pick_val[p] - maximum);
        const float w = raw / denom * d.scale;
        ws.ids[slot] = id;
        ws.weights[slot] = w;
        if (route_dense) route_dense[id] = w;
    }
    // The shared expert's weight: its gate's Sigmoid activation, 0.5 (tanh(v/2) + 1)
    // (recipe.rs:22662-22668), or 1 when it has no gate.
    if (lane == 0 && d.hidden_shared > 0)
        ws.weights[d.top] = d.shared_gated ? 0.5f * (tanhf(0.5f * ws.logits[E]) + 1.0f) : 1.0f;
}

template <int FMT, bool XF32>
__global__ void __launch_bounds__(256) moe_glu_kernel(MoeDims d, MoeBank gate, MoeBank up, MoeBank gate_sh,
                                                       MoeBank up_sh, const void* x, MoeWorkspace ws, int G) {
    constexpr int XP = Traits<FMT>::XP;
    extern __shared__ uint4 smem[];
    const int nch = gate.P.nch;
    uint4* xd = smem;
    uint4* xb = smem + XP * nch;
    stage_all<FMT, XF32>(nch, d.d_model, x, 0, 1, xd, reinterpret_cast<float*>(xb));
    __syncthreads();
    const int lane = threadIdx.x & 63, g = lane & (G - 1), sub = lane / G;
    const int wpb = blockDim.x >> 6, wave = threadIdx.x >> 6;
    const int routed = d.top * d.hidden;
    const int total_rows = routed + d.hidden_shared;
    const int rows_per_wave = 64 / G;
    const int tiles = (total_rows + rows_per_wave - 1) / rows_per_wave;
    for (int tile = blockIdx.x * wpb + wave; tile < tiles; tile += gridDim.x * wpb) {
        const int r = tile * rows_per_wave + sub;
        if (r >= total_rows) continue;  // whole lane group idles; reductions stay inside the group
        Planes pg, pu;
        int64_t rg, ru;
        if (r < routed) {
            const int s = r / d.hidden, f = r % d.hidden;
            const int64_t e = ws.ids[s];
            pg = gate.P;
            pu = up.P;
            rg = e * gate.rows + f;
            ru = e * up.rows + f;
        } else {
            const int f = r - routed;
            pg = gate_sh.P;
            pu = up_sh.P;
            rg = f;
            ru = f;
        }
        float ag = 0.f, au = 0.f;
        for (int c = g; c < nch; c += G) {
            ChunkData<FMT> dg, du;
            load_chunk<FMT>(pg, rg, c, dg);
            load_chunk<FMT>(pu, ru, c, du);
            uint4 xv[1][XP];
            uint4 bv[1][2];
#pragma unroll
            for (int j = 0; j < XP; ++j) xv[0][j] = xd[j * nch + c];
            bv[0][0] = xb[c];
            bv[0][1] = xb[nch + c];
            dot_int<FMT, 1>(dg, c, xv, bv, &ag);
            dot_int<FMT, 1>(du, c, xv, bv, &au);
        }
        ag = group_sum(ag, G);
        au = group_sum(au, G);
        if (g == G - 1) ws.h[r] = ag * sigmoidf_dev(ag) * au;
    }
}

template <int FMT>
__global__ void __launch_bounds__(256) moe_down_kernel(MoeDims d, MoeBank down, MoeBank down_sh, MoeWorkspace ws,
                                                        float* y, int G) {
    constexpr int CW = Traits<FMT>::CW, XP = Traits<FMT>::XP;
    extern __shared__ uint4 smem[];
    const int K = d.top * d.hidden + d.hidden_shared;
    const int nch = K / CW;            // chunks of all slots back to back
    const int cps = d.hidden / CW;     // chunks per routed slot
    const int routed_ch = d.top * cps;
    uint4* xd = smem;
    uint4* xb = smem + XP * nch;
    stage_all<FMT, true>(nch, K, ws.h, 0, 1, xd, reinterpret_cast<float*>(xb));
    __syncthreads();
    const int lane = threadIdx.x & 63, g = lane & (G - 1), sub = lane / G;
    const int wpb = blockDim.x >> 6, wave = threadIdx.x >> 6;
    const int rows_per_wave = 64 / G;
    const int tiles = (d.d_model + rows_per_wave - 1) / rows_per_wave;
    for (int tile = blockIdx.x * wpb + wave; tile < tiles; tile += gridDim.x * wpb) {
        const int n = tile * rows_per_wave + sub;
        if (n >= d.d_model) continue;
        float acc = 0.f;
        for (int c = g; c < nch; c += G) {
            ChunkData<FMT> cd;
            float w;
            int lc;
            if (c < routed_ch) {
                const int s = c / cps;
                lc = c - s * cps;
                load_chunk<FMT>(down.P, (int64_t)ws.ids[s] * down.rows + n, lc, cd);
                w = ws.weights[s];
            } else {
                lc = c - routed_ch;
                load_chunk<FMT>(down_sh.P, n, lc, cd);
                w = ws.weights[d.top];
            }
            uint4 xv[1][XP];
            uint4 bv[1][2];
#pragma unroll
            for (int j = 0; j < XP; ++j) xv[0][j] = xd[j * nch + c];
            bv[0][0] = xb[c];
            bv[0][1] = xb[nch + c];
            float part = 0.f;
            dot_int<FMT, 1>(cd, lc, xv, bv, &part);
            acc = fmaf(w, part, acc);
        }
        acc = group_sum(acc, G);
        if (g == G - 1) y[n] = acc;
    }
}

hipError_t launch_moe_topk(const MoeDims& d, MoeWorkspace ws, float* route_dense, hipStream_t stream) {
    if (d.experts > 64 * kTopkSlots || d.top > 64 || d.top < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(moe_topk_kernel, dim3(1), dim3(64), 0, stream, d, ws, route_dense);
    return hipGetLastError();
}

static int lanes_for(int64_t nch) {
    int G = 64;
    while (G > 8 && G > nch) G >>= 1;
    return G;
}

template <int FMT>
static hipError_t glu_fmt(int xtype, const MoeDims& d, const MoeBank& gate, const MoeBank& up, const MoeBank& gate_sh,
                          const MoeBank& up_sh, const void* x, MoeWorkspace ws, int cus, hipStream_t stream) {
    const int nch = gate.P.nch;
    const int G = lanes_for(nch);
    const int total_rows = d.top * d.hidden + d.hidden_shared;
    const int rows_per_block = 4 * (64 / G);
    int grid = (total_rows + rows_per_block - 1) / rows_per_block;
    if (grid > cus * 8) grid = cus * 8;
    const size_t lds = stage_bytes_int(FMT, 1, nch);
    if (lds > 65536) {
        hipError_t e = hipFuncSetAttribute(xtype == 0 ? reinterpret_cast<const void*>(&moe_glu_kernel<FMT, true>)
                                                       : reinterpret_cast<const void*>(&moe_glu_kernel<FMT, false>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    if (xtype == 0)
        hipLaunchKernelGGL((moe_glu_kernel<FMT, true>), dim3(grid), dim3(256), lds, stream, d, gate, up, gate_sh, up_sh,
                           x, ws, G);
    else
        hipLaunchKernelGGL((moe_glu_kernel<FMT, false>), dim3(grid), dim3(256), lds, stream, d, gate, up, gate_sh,
                           up_sh, x, ws, G);
    return hipGetLastError();
}

hipError_t launch_moe_glu(int fmt, int xtype, const MoeDims& d, const MoeBank& gate, const MoeBank& up,
                          const MoeBank& gate_sh, const MoeBank& up_sh, const void* x, MoeWorkspace ws, int cus,
                          hipStream_t stream) {
    switch (fmt) {
        case Q4_0: return glu_fmt<Q4_0>(xtype, d, gate, up, gate_sh, up_sh, x, ws, cus, stream);
        case Q8_0: return glu_fmt<Q8_0>(xtype, d, gate, up, gate_sh, up_sh, x, ws, cus, stream);
        case Q4_K: return glu_fmt<Q4_K>(xtype, d, gate, up, gate_sh, up_sh, x, ws, cus, stream);
        case Q6_K: return glu_fmt<Q6_K>(xtype, d, gate, up, gate_sh, up_sh, x, ws, cus, stream);
        default: return hipErrorInvalidValue;
    }
}

template <int FMT>
static hipError_t down_fmt(const MoeDims& d, const MoeBank& down, const MoeBank& down_sh, MoeWorkspace ws, float* y,
                           int cus, hipStream_t stream) {
    constexpr int CW = Traits<FMT>::CW;
    const int nch = (d.top * d.hidden + d.hidden_shared) / CW;
    const int G = lanes_for(nch);
    const int rows_per_block = 4 * (64 / G);
    int grid = (d.d_model + rows_per_block - 1) / rows_per_block;
    if (grid > cus * 8) grid = cus * 8;
    const size_t lds = stage_bytes_int(FMT, 1, nch);
    if (lds > 65536) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&moe_down_kernel<FMT>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(moe_down_kernel<FMT>, dim3(grid), dim3(256), lds, stream, d, down, down_sh, ws, y, G);
    return hipGetLastError();
}

hipError_t launch_moe_down(int fmt, const MoeDims& d, const MoeBank& down, const MoeBank& down_sh, MoeWorkspace ws,
                           float* y, int cus, hipStream_t stream) {
    switch (fmt) {
        case Q4_0: return down_fmt<Q4_0>(d, down, down_sh, ws, y, cus, stream);
        case Q8_0: return down_fmt<Q8_0>(d, down, down_sh, ws, y, cus, stream);
        case Q4_K: return down_fmt<Q4_K>(d, down, down_sh, ws, y, cus, stream);
        case Q6_K: return down_fmt<Q6_K>(d, down, down_sh, ws, y, cus, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace rq
