// gguf_moe block on gfx950: one position, or a batch of positions (prefill)
// along the launches' y dimension, each with its own routing.
//
// Reference: lower_gguf_moe (recipe.rs:23415-23459) emits router Contraction ->
// TopK -> ExpertIn(gate), ExpertIn(up) -> silu(gate)*up -> ExpertOut(down), and a
// shared expert as a one-expert bank weighted by its gate; the device bodies
// are topk_forward_wave_body (amd-nv-cpu.ll:4489-4652) and packed_lanes_body
// modes 1/2 (amd-nv-cpu.ll:2897-2986, 3041-3086).
//
// Here the router and the shared expert's gate run as one F16 matvec, then:
//   moe_glu   every wave first routes the position (a radix select of the k
//             best selection keys, the lower expert on a tie; the routing
//             weights; slots in ascending expert id), then one lane group per
//             (slot, hidden row) reads the gate and up rows of the slot's
//             expert together against x staged in LDS, and act(gate) * up is
//             written per slot (routed slots, then shared);
//   moe_down  one lane group per output row: its lanes walk the chunks of every
//             slot's down row (K = all slots' hidden widths back to back, h staged
//             in LDS), scale each chunk by its slot's weight, and reduce across
//             lanes; no atomics, no second pass.
#include "act.h"
#include "moe.h"
#include "stage.h"

namespace rq {

constexpr int kMoeThreads = 256;  // workgroup size of the MoE kernels (four waves)
constexpr int kMoeOwnRouteMax = 2;  // positions per launch up to which every wave routes on its own

static size_t al(size_t v) { return (v + 255) & ~size_t(255); }
static bool env_flag(const char* name, bool fallback) {
    const char* v = getenv(name);
    return v && *v ? *v != '0' : fallback;
}

// Workgroups per position of a launch: at most eight per CU over the whole
// batch (each workgroup routes or stages its position once, so a batch of
// many positions walks several tiles per wave rather than repeating that
// work in more workgroups), and at least one.
static int batch_grid_cap(int cus, int m) {
    const int cap = cus * 8 / (m > 0 ? m : 1);
    return cap > 1 ? cap : 1;
}

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

// @sigmoid of the router's scoring (amd-nv-cpu.ll:5007-5009): 1 / (1 + exp(-v)).
__device__ __forceinline__ float sigmoidf_dev(float v) { return 1.0f / (1.0f + expf(-v)); }

// The workspace of position p of a batch.
__device__ __forceinline__ MoeWorkspace position_ws(MoeWorkspace ws, int64_t stride_bytes, int p) {
    const int64_t o = stride_bytes * p;
    ws.logits = reinterpret_cast<float*>(reinterpret_cast<char*>(ws.logits) + o);
    ws.ids = reinterpret_cast<int*>(reinterpret_cast<char*>(ws.ids) + o);
    ws.weights = reinterpret_cast<float*>(reinterpret_cast<char*>(ws.weights) + o);
    ws.h = reinterpret_cast<float*>(reinterpret_cast<char*>(ws.h) + o);
    return ws;
}

// (value, index) pair of the better expert: the higher score, the lower id on a tie.
__device__ __forceinline__ void better_of(float& v, int& i, float pv, int pi) {
    const bool take = pv > v || (pv == v && pi < i);
    v = take ? pv : v;
    i = take ? pi : i;
}

// One argmax step against the lane DPP control CTRL names (rows in ROW_MASK);
// a lane without a source keeps its own pair.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ void argmax_dpp(float& v, int& i) {
    const int vb = __builtin_bit_cast(int, v);
    const float pv = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(vb, vb, CTRL, ROW_MASK, 0xf, false));
    const int pi = __builtin_amdgcn_update_dpp(i, i, CTRL, ROW_MASK, 0xf, false);
    better_of(v, i, pv, pi);
}

// The best (value, index) of the wave, in every lane: pairs within quads,
// half rows and rows, then rows 0-1 into row 1, rows 2-3 into row 3 and row 1
// into row 3 (the DPP pattern of a wave scan), read back from lane 63.
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
    argmax_dpp<0xB1, 0xF>(v, i);   // quad_perm [1,0,3,2]
    argmax_dpp<0x4E, 0xF>(v, i);   // quad_perm [2,3,0,1]
    argmax_dpp<0x141, 0xF>(v, i);  // row_half_mirror
    argmax_dpp<0x140, 0xF>(v, i);  // row_mirror
    argmax_dpp<0x142, 0xA>(v, i);  // row_bcast:15
    argmax_dpp<0x143, 0xC>(v, i);  // row_bcast:31
    v = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
    i = __builtin_amdgcn_readlane(i, 63);
}

// Sum over the wave in a fixed DPP order, in every lane.
__device__ __forceinline__ float wave_sum_fixed(float v) {
    v = group_sum(v, 64);
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Top-k routing (topk_forward_body semantics, amd-nv-cpu.ll:4486-4716) on one
// wave. The selection keys sit in registers (expert lane + 64 j in key[j]) as
// order-preserving 32-bit patterns: the router score itself, or with a
// selection bias (topk_key, amd-nv-cpu.ll:4653-4660) the expert's probability
// (its sigmoid, or exp(score - max) / total over every expert) plus its bias,
// formed in fp32. A radix select over the 32 key bits (one ballot and
// population count per register per bit) finds the k-th largest key T; the
// experts above T are kept, and of those equal to T the lowest ids, so a tie
// goes to the lower expert. Slots are the kept experts in ascending id,
// counted from the ballots. The weights come from the unbiased scores. The
// picked ids go to the wave's `slot_ids` (LDS); with `publish` the wave also
// writes the routing (ids, weights, the shared expert's weight, the dense
// routing plane) to the workspace. Sums run in a fixed order, so the weights
// are deterministic.
constexpr int kTopkMaxExperts = 2048;

__device__ __forceinline__ uint32_t order_key(float f) {
    const uint32_t u = __builtin_bit_cast(uint32_t, f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Lanes below this one whose bit is set in `mask`.
__device__ __forceinline__ int lanes_below(uint64_t mask) {
    return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

template <int S>
__device__ __forceinline__ void route_wave(const MoeDims& d, const MoeWorkspace& ws, float* route_dense, bool publish,
                                           int* slot_ids) {
    const int lane = threadIdx.x & 63;
    const int E = d.experts, k = d.top;
    const bool sigmoid = d.scoring != 0, renorm = d.renormalize != 0;
    float v[S];
    uint32_t key[S];
#pragma unroll
    for (int j = 0; j < S; ++j) {
        const int e = lane + 64 * j;
        v[j] = ws.logits[e < E ? e : E - 1];
        key[j] = e < E ? order_key(v[j]) : 0u;  // an absent expert ranks below every score
    }
    const float shared_logit = ws.logits[E];  // read early; used only with a gated shared expert
    if (__builtin_expect(d.sel_bias != nullptr, 0)) {
        float bias[S];
#pragma unroll
        for (int j = 0; j < S; ++j) {
            const int e = lane + 64 * j;
            bias[j] = d.sel_bias[e < E ? e : E - 1];
        }
        // probability over every expert, plus the bias
        float am = -INFINITY;
#pragma unroll
        for (int j = 0; j < S; ++j)
            if (lane + 64 * j < E) am = fmaxf(am, v[j]);
        {
            int ii = 0;
            wave_argmax(am, ii);
        }
        float at = 0.f;
#pragma unroll
        for (int j = 0; j < S; ++j)
            if (lane + 64 * j < E) at += sigmoid ? sigmoidf_dev(v[j]) : expf(v[j] - am);
        const float all_total = wave_sum_fixed(at);
#pragma unroll
        for (int j = 0; j < S; ++j) {
            const float raw = sigmoid ? sigmoidf_dev(v[j]) : expf(v[j] - am);
            const float prob = sigmoid ? raw : raw / all_total;
            key[j] = lane + 64 * j < E ? order_key(prob + bias[j]) : 0u;
        }
    }
    // T = the largest key with at least k keys >= T. Once exactly k keys are
    // >= T the kept set is known (it is {key >= T}, as it would be at the
    // final T), so the remaining bits are skipped.
    uint32_t T = 0;
    for (int bit = 31; bit >= 0; --bit) {
        const uint32_t cand = T | (1u << bit);
        int cnt = 0;
#pragma unroll
        for (int j = 0; j < S; ++j) cnt += __popcll(__ballot(key[j] >= cand));
        if (cnt >= k) {
            T = cand;
            if (cnt == k) break;
        }
    }
    int above = 0;
#pragma unroll
    for (int j = 0; j < S; ++j) above += __popcll(__ballot(key[j] > T));
    // keep every key above T and the (k - above) lowest-id keys equal to T;
    // slot = kept experts of lower id
    int need = k - above, kept_before = 0;
    bool kept[S];
    int slot[S];
#pragma unroll
    for (int j = 0; j < S; ++j) {
        const uint64_t eq = __ballot(key[j] == T);
        const bool take_eq = key[j] == T && lanes_below(eq) < need;
        kept[j] = key[j] > T || take_eq;
        const int taken_eq = __popcll(eq) < need ? __popcll(eq) : need;
        need -= taken_eq;
        const uint64_t km = __ballot(kept[j]);
        slot[j] = kept_before + lanes_below(km);
        kept_before += __popcll(km);
    }
    // the slots first: the expert loads wait for them
#pragma unroll
    for (int j = 0; j < S; ++j)
        if (kept[j]) slot_ids[slot[j]] = lane + 64 * j;
    if (publish) {
        // maximum and total over the kept experts (renormalized) or over all
        float m = -INFINITY;
#pragma unroll
        for (int j = 0; j < S; ++j)
            if ((renorm ? kept[j] : lane + 64 * j < E)) m = fmaxf(m, v[j]);
        float mx = m;
        {
            int ii = 0;
            wave_argmax(mx, ii);
        }
        float t = 0.f;
#pragma unroll
        for (int j = 0; j < S; ++j)
            if ((renorm ? kept[j] : lane + 64 * j < E)) t += sigmoid ? sigmoidf_dev(v[j]) : expf(v[j] - mx);
        const float total = wave_sum_fixed(t);
        const float denom = (renorm || !sigmoid) ? total : 1.0f;
#pragma unroll
        for (int j = 0; j < S; ++j) {
            const int e = lane + 64 * j;
            if (e >= E) continue;
            const float raw = sigmoid ? sigmoidf_dev(v[j]) : expf(v[j] - mx);
            const float w = raw / denom * d.scale;
            if (kept[j]) {
                ws.ids[slot[j]] = e;
                ws.weights[slot[j]] = w;
            }
            if (route_dense) route_dense[e] = kept[j] ? w : 0.f;
        }
        // The shared expert's weight: its gate's activation (SharedExpert::Gated,
        // recipe.rs:23440-23452), or 1 when it has no gate.
        if (lane == 0 && d.hidden_shared > 0)
            ws.weights[k] = d.shared_gated ? act_apply_likely_sigmoid(d.shared_gate_act, d.act_factor, shared_logit) : 1.0f;
    }
}

// RING (batches): two buffers of weights, the next tile's requested before
// the current one is computed. One or two positions run one tile per wave,
// where the single buffer holds fewer registers and measured faster.
//
// Each row's gate and up sums add one partial per chunk (each chunk's dot
// formed from zero), in the chunk order of G lanes per row pair (lane g:
// chunks g, g + G, ...). GSPLIT (one position) runs 2G lanes per row pair with
// those sums: lane g < G adds its chunk's partials and then, through a lane
// swap, those of lane g + G (chunk g + G), so every row carries the bits of
// the G-lane form with twice the lanes.
template <int FMT, bool XF32, int S, bool RING, bool GSPLIT = false>
__global__ void __launch_bounds__(kMoeThreads) moe_glu_kernel(MoeDims d, MoeBank gate, MoeBank up, MoeBank gate_sh,
                                                       MoeBank up_sh, const void* x, MoeWorkspace ws, float* route_dense,
                                                       int G, MoeBatch batch) {
    constexpr int XP = Traits<FMT>::XP;
    // position blockIdx.y of the batch
    x = static_cast<const char*>(x) + batch.x_stride * blockIdx.y;
    ws = position_ws(ws, batch.ws_stride, (int)blockIdx.y);
    if (route_dense) route_dense += batch.route_stride * blockIdx.y;
    extern __shared__ uint4 smem[];
    __shared__ int slot_ids_all[4][64];
    const int nch = gate.P.nch;
    uint4* xd = smem;
    uint4* xb = smem + XP * nch;
    const int lane = threadIdx.x & 63, g = lane & (G - 1), sub = lane / G;
    const int wpb = kMoeThreads >> 6, wave = threadIdx.x >> 6;
    const int routed = d.top * d.hidden;
    const int total_rows = routed + d.hidden_shared;
    const int rows_per_wave = 64 / G;
    const int tiles = (total_rows + rows_per_wave - 1) / rows_per_wave;
    // The position is routed here (a few microseconds of one wave, instead of
    // a launch and a round trip through memory); the first wave of the first
    // workgroup also writes the routing out for the down kernel. For one or
    // two positions every wave routes on its own and none waits; for more,
    // where the launch holds many workgroups per position, the first wave
    // routes for its workgroup and the others read its slots after a barrier.
    // (RING is chosen for exactly the launches of more than two positions.)
    int* const slot_ids = slot_ids_all[RING ? 0 : wave];
    // the activation loads go out first, so that they land while the position is routed
    const bool multi = stage_items<FMT>(nch, 1) <= kStageNJ * kMoeThreads;
    StageItem<XF32> it[kStageNJ];
    if (multi) stage_multi_issue<FMT, XF32>(nch, d.d_model, x, 0, 1, kMoeThreads, it);
    if (!RING || wave == 0) route_wave<S>(d, ws, route_dense, blockIdx.x == 0 && wave == 0, slot_ids);
    if constexpr (RING) __syncthreads();
    // Row r of the gate/up stack: hidden row f of routed slot s, or of the shared expert.
    auto fetch = [&](int r, int c, ChunkData<FMT>& dg, ChunkData<FMT>& du) {
        r = r < total_rows ? r : total_rows - 1;
        c = c < nch ? c : nch - 1;
        if (r < routed) {
            const int s = r / d.hidden, f = r % d.hidden;
            const int64_t e = slot_ids[s];
            load_chunk<FMT>(gate.P, e * gate.rows + f, c, dg);
            load_chunk<FMT>(up.P, e * up.rows + f, c, du);
        } else {
            load_chunk<FMT>(gate_sh.P, r - routed, c, dg);
            load_chunk<FMT>(up_sh.P, r - routed, c, du);
        }
    };
    int tile = blockIdx.x * wpb + wave;
    const int stride = gridDim.x * wpb;
    // the first tile's weights are requested before the activations are staged
    ChunkData<FMT> dg0, du0, dg1, du1;
    fetch((tile < tiles ? tile : tiles - 1) * rows_per_wave + sub, g, dg0, du0);
    __shared__ int wave_flags[kMoeThreads / 64];
    publish_outliers(multi ? stage_multi_finish<FMT, XF32>(nch, d.d_model, 1, kMoeThreads, it, xd, reinterpret_cast<float*>(xb))
                           : stage_all<FMT, XF32>(nch, d.d_model, x, 0, 1, kMoeThreads, xd, reinterpret_cast<float*>(xb)),
                     wave_flags);
    __syncthreads();
    const bool outliers = read_outliers(wave_flags, kMoeThreads);
    // one chunk's gate and up partials, each formed from zero
    auto partials = [&](int c, const ChunkData<FMT>& dg, const ChunkData<FMT>& du, float& pg, float& pu) {
        uint4 xv[XP];
        uint4 bv[2];
#pragma unroll
        for (int j = 0; j < XP; ++j) xv[j] = xd[j * nch + c];
        bv[0] = xb[c];
        bv[1] = xb[nch + c];
        pg = 0.f;
        pu = 0.f;
        dot_int<FMT>(dg, c, xv, bv, pg);
        dot_int<FMT>(du, c, xv, bv, pu);
        if (__builtin_expect(outliers && wave_has_outlier(bv[0]), 0)) {
            dot_outliers<FMT>(dg, c, xb + c, nch, pg);
            dot_outliers<FMT>(du, c, xb + c, nch, pu);
        }
    };
    if constexpr (GSPLIT) {
        const int GE = G >> 1;  // the lanes whose sums every row carries
        bool fetched = true;
        for (; tile < tiles; tile += stride) {
            const int r = tile * rows_per_wave + sub;
            float ag = 0.f, au = 0.f;
            for (int c0 = 0; c0 < nch; c0 += G) {
                const int c = c0 + g;
                if (!fetched) fetch(r, c, dg0, du0);
                fetched = false;
                float pg = 0.f, pu = 0.f;
                if (c < nch) partials(c, dg0, du0, pg, pu);
                // (lo, hi): lane g's and lane g + GE's partials, in every lane g < GE
                float gl = pg, gh = pg, ul = pu, uh = pu;
                if (GE == 16) {
                    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(gl), "+v"(gh));
                    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(ul), "+v"(uh));
                } else {
                    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(gl), "+v"(gh));
                    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(ul), "+v"(uh));
                }
                if (g < GE) {
                    if (c < nch) {
                        ag += gl;
                        au += ul;
                    }
                    if (c + GE < nch) {
                        ag += gh;
                        au += uh;
                    }
                }
            }
            ag = group_sum(ag, GE);
            au = group_sum(au, GE);
            if (r < total_rows && g == GE - 1) ws.h[r] = act_apply_likely_silu(d.activation, d.act_factor, ag) * au;
        }
        return;
    }
    if constexpr (!RING) {
        bool fetched = true;
        for (; tile < tiles; tile += stride) {
            const int r = tile * rows_per_wave + sub;
            float ag = 0.f, au = 0.f;
            for (int c = g; c < nch; c += G) {
                if (!fetched) fetch(r, c, dg0, du0);
                fetched = false;
                float pg, pu;
                partials(c, dg0, du0, pg, pu);
                ag += pg;
                au += pu;
            }
            ag = group_sum(ag, G);
            au = group_sum(au, G);
            if (r < total_rows && g == G - 1) ws.h[r] = act_apply_likely_silu(d.activation, d.act_factor, ag) * au;
        }
        return;
    }
    // One tile from the buffers (dg, du), whose first chunk is loaded; the
    // next tile's first chunk goes to (ng, nu) before this one is computed.
    auto step = [&](int t, ChunkData<FMT>& dg, ChunkData<FMT>& du, ChunkData<FMT>& ng, ChunkData<FMT>& nu) {
        const int r = t * rows_per_wave + sub;
        if (t + stride < tiles) fetch((t + stride) * rows_per_wave + sub, g, ng, nu);
        float ag = 0.f, au = 0.f;
        for (int c = g; c < nch; c += G) {
            if (c != g) fetch(r, c, dg, du);  // a row longer than one chunk per lane
            float pg, pu;
            partials(c, dg, du, pg, pu);
            ag += pg;
            au += pu;
        }
        ag = group_sum(ag, G);
        au = group_sum(au, G);
        if (r < total_rows && g == G - 1) ws.h[r] = act_apply_likely_silu(d.activation, d.act_factor, ag) * au;
    };
    while (tile < tiles) {
        step(tile, dg0, du0, dg1, du1);
        tile += stride;
        if (tile >= tiles) break;
        step(tile, dg1, du1, dg0, du0);
        tile += stride;
    }
}

// TAIL (with SPLIT, rows of 65-72 chunks): eight row waves and a ninth that
// forms the partials of the chunks past 64 for all eight rows (below).
// SPLIT (one or two positions, G = 32): one row per wave, its lanes taking
// chunks lane, lane + 64, ... as 64 lanes would, with the sums formed in the
// order of 32 lanes per row (lane g adds chunk g + 64 s, then lane g + 32's
// chunk g + 32 + 64 s, through a 32-lane swap), so that every row carries the
// bits of the 32-lane form with twice the waves.
template <int FMT, bool RING, int BT = kMoeThreads, bool SPLIT = false, bool TAIL = false>
__global__ void __launch_bounds__(BT) moe_down_kernel(MoeDims d, MoeBank down, MoeBank down_sh, MoeWorkspace ws,
                                                        float* y, int G, MoeBatch batch) {
    constexpr int CW = Traits<FMT>::CW, XP = Traits<FMT>::XP;
    ws = position_ws(ws, batch.ws_stride, (int)blockIdx.y);
    y += batch.y_stride * blockIdx.y;
    extern __shared__ uint4 smem[];
    const int K = d.top * d.hidden + d.hidden_shared;
    const int nch = K / CW;            // chunks of all slots back to back
    const int cps = d.hidden / CW;     // chunks per routed slot
    const int routed_ch = d.top * cps;
    uint4* xd = smem;
    uint4* xb = smem + XP * nch;
    static_assert(!(SPLIT && RING), "the split form is for one or two positions");
    const int lane = threadIdx.x & 63, g = SPLIT ? lane : lane & (G - 1), sub = SPLIT ? 0 : lane / G;
    // TAIL: the last wave takes chunks 64.. of the other waves' rows (its lane
    // l: row l / 8, chunk 64 + l % 8)
    const int wpb = (BT >> 6) - (TAIL ? 1 : 0), wave = threadIdx.x >> 6;
    const bool tail_wave = TAIL && wave == wpb;
    const int rows_per_wave = SPLIT ? 1 : 64 / G;
    const int tiles = (d.d_model + rows_per_wave - 1) / rows_per_wave;
    // Chunk c of output row n: chunk lc of slot s's expert down row, or of the shared expert's.
    auto fetch = [&](int n, int c, ChunkData<FMT>& cd, float& w, int& lc) {
        n = n < d.d_model ? n : d.d_model - 1;
        c = c < nch ? c : nch - 1;
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
    };
    int tile = blockIdx.x * wpb + wave;
    const int stride = gridDim.x * wpb;
    // The slot activations' loads go out first (they do not depend on the
    // routing), then the first tile's weights (which wait for the slot ids);
    // all of them are in flight before any activation is encoded.
    const bool multi = stage_items<FMT>(nch, 1) <= kStageNJ * BT;
    StageItem<true> it[kStageNJ];
    if (multi) stage_multi_issue<FMT, true>(nch, K, ws.h, 0, 1, BT, it);
    ChunkData<FMT> cd0, cd1;
    float w0, w1;
    int lc0, lc1;
    if (tail_wave)
        fetch(blockIdx.x * wpb + (lane >> 3), 64 + (lane & 7), cd0, w0, lc0);
    else
        fetch((tile < tiles ? tile : tiles - 1) * rows_per_wave + sub, g, cd0, w0, lc0);
    __shared__ int wave_flags[BT / 64];
    publish_outliers(multi ? stage_multi_finish<FMT, true>(nch, K, 1, BT, it, xd, reinterpret_cast<float*>(xb))
                           : stage_all<FMT, true>(nch, K, ws.h, 0, 1, BT, xd, reinterpret_cast<float*>(xb)),
                     wave_flags);
    __syncthreads();
    const bool outliers = read_outliers(wave_flags, BT);
    if constexpr (TAIL) {
        // Rows of 65-72 chunks, one per wave, one tile per wave (the launch
        // covers every row): the tail wave forms the partials of chunks 64..
        // and hands them over through LDS, so that no wave takes a second
        // step and the staging needs one item per thread. Each row's sum is
        // the SPLIT form's, operation for operation: lane g < 32 adds chunk g,
        // then chunk g + 32, then (g < nch - 64) chunk 64 + g.
        __shared__ float tail_part[64];
        __shared__ float tail_w[8];
        const int c = tail_wave ? 64 + (lane & 7) : lane;
        float part = 0.f;
        if (c < nch) {
            uint4 xv[XP];
            uint4 bv[2];
#pragma unroll
            for (int j = 0; j < XP; ++j) xv[j] = xd[j * nch + c];
            bv[0] = xb[c];
            bv[1] = xb[nch + c];
            dot_int<FMT>(cd0, lc0, xv, bv, part);
            if (__builtin_expect(outliers && wave_has_outlier(bv[0]), 0)) dot_outliers<FMT>(cd0, lc0, xb + c, nch, part);
        }
        float acc = 0.f;
        if (tail_wave) {
            tail_part[lane] = part;
            if (lane < 8) tail_w[lane] = w0;
        } else {
            float pu = part, wu = w0, pl = part, wl = w0;
            asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(pl), "+v"(pu));
            asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(wl), "+v"(wu));
            if (lane < 32) {
                acc = fmaf(w0, part, acc);
                if (c + 32 < nch) acc = fmaf(wu, pu, acc);
            }
        }
        __syncthreads();
        if (tail_wave) return;
        if (64 + lane < nch && lane < 8) acc = fmaf(tail_w[lane], tail_part[8 * wave + lane], acc);
        acc = group_sum(acc, 32);
        const int n = blockIdx.x * wpb + wave;
        if (n < d.d_model && lane == 31) y[n] = acc;
        return;
    }
    if constexpr (SPLIT) {
        bool fetched = true;
        for (; tile < tiles; tile += stride) {
            const int n = tile;
            float acc = 0.f;
            for (int c0 = 0; c0 < nch; c0 += 64) {
                const int c = c0 + lane;
                if (!fetched) fetch(n, c, cd0, w0, lc0);
                fetched = false;
                float part = 0.f;
                if (c < nch) {
                    uint4 xv[XP];
                    uint4 bv[2];
#pragma unroll
                    for (int j = 0; j < XP; ++j) xv[j] = xd[j * nch + c];
                    bv[0] = xb[c];
                    bv[1] = xb[nch + c];
                    dot_int<FMT>(cd0, lc0, xv, bv, part);
                    if (__builtin_expect(outliers && wave_has_outlier(bv[0]), 0)) dot_outliers<FMT>(cd0, lc0, xb + c, nch, part);
                }
                // lane + 32's chunk and weight, in every lane below 32
                float pu = part, wu = w0, pl = part, wl = w0;
                asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(pl), "+v"(pu));
                asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(wl), "+v"(wu));
                if (lane < 32) {
                    if (c < nch) acc = fmaf(w0, part, acc);
                    if (c + 32 < nch) acc = fmaf(wu, pu, acc);
                }
            }
            acc = group_sum(acc, 32);
            if (n < d.d_model && lane == 31) y[n] = acc;
        }
        return;
    }
    if constexpr (!RING) {
        bool fetched = true;
        for (; tile < tiles; tile += stride) {
            const int n = tile * rows_per_wave + sub;
            float acc = 0.f;
            for (int c = g; c < nch; c += G) {
                if (!fetched) fetch(n, c, cd0, w0, lc0);
                fetched = false;
                uint4 xv[XP];
                uint4 bv[2];
#pragma unroll
                for (int j = 0; j < XP; ++j) xv[j] = xd[j * nch + c];
                bv[0] = xb[c];
                bv[1] = xb[nch + c];
                float part = 0.f;
                dot_int<FMT>(cd0, lc0, xv, bv, part);
                if (__builtin_expect(outliers && wave_has_outlier(bv[0]), 0)) dot_outliers<FMT>(cd0, lc0, xb + c, nch, part);
                acc = fmaf(w0, part, acc);
            }
            acc = group_sum(acc, G);
            if (n < d.d_model && g == G - 1) y[n] = acc;
        }
        return;
    }
    // One tile from (cd, w, lc), whose first chunk is loaded; the next tile's
    // first chunk goes to (nd, nw, nlc) before this one is computed.
    auto step = [&](int t, ChunkData<FMT>& cd, float& w, int& lc, ChunkData<FMT>& nd, float& nw, int& nlc) {
        const int n = t * rows_per_wave + sub;
        if (t + stride < tiles) fetch((t + stride) * rows_per_wave + sub, g, nd, nw, nlc);
        float acc = 0.f;
        for (int c = g; c < nch; c += G) {
            if (c != g) fetch(n, c, cd, w, lc);  // the lane's later chunks of the row, in turn
            uint4 xv[XP];
            uint4 bv[2];
#pragma unroll
            for (int j = 0; j < XP; ++j) xv[j] = xd[j * nch + c];
            bv[0] = xb[c];
            bv[1] = xb[nch + c];
            float part = 0.f;
            dot_int<FMT>(cd, lc, xv, bv, part);
            if (__builtin_expect(outliers && wave_has_outlier(bv[0]), 0)) dot_outliers<FMT>(cd, lc, xb + c, nch, part);
            acc = fmaf(w, part, acc);
        }
        acc = group_sum(acc, G);
        if (n < d.d_model && g == G - 1) y[n] = acc;
    };
    while (tile < tiles) {
        step(tile, cd0, w0, lc0, cd1, w1, lc1);
        tile += stride;
        if (tile >= tiles) break;
        step(tile, cd1, w1, lc1, cd0, w0, lc0);
        tile += stride;
    }
}

static int lanes_for(int64_t nch) {
    int G = 64;
    while (G > 8 && G > nch) G >>= 1;
    return G;
}

template <int FMT, bool XF32, int S>
static hipError_t glu_launch(const MoeDims& d, const MoeBank& gate, const MoeBank& up, const MoeBank& gate_sh,
                             const MoeBank& up_sh, const void* x, MoeWorkspace ws, float* route_dense,
                             const MoeBatch& b, int cus, hipStream_t stream) {
    const int nch = gate.P.nch;
    // Lanes per gate/up row pair: half of one chunk per lane, so that each
    // workgroup's staging of x serves twice the rows (constant over batch
    // sizes: batches stay bit-identical to one-position calls). Measured on
    // the gguf_moe workload (d_model 2048, 32 chunks), us per step at 1 / 4 /
    // 16 positions: 20.6 / 37.9 / 82.5 at 32 lanes, 20.7 / 36.1 / 81.3 at 16,
    // 21.8 / 32.5 / 85.0 at 8. RQMV_MOE_GLU_G overrides it.
    const char* glu_genv = getenv("RQMV_MOE_GLU_G");
    int G = lanes_for(nch);
    if (G > 8) G >>= 1;
    if (glu_genv && *glu_genv) {
        const int g = atoi(glu_genv);
        if (g == 8 || g == 16 || g == 32 || g == 64) G = g;
    }
    // At one position, twice the lanes with the same sums (GSPLIT): 32 lanes
    // per row pair in the 16-lane sum order, 16.78 -> 16.43 us per step (two
    // alternating pairs; two and four positions unchanged with the partial
    // sums). RQMV_MOE_GLU_SPLIT=0/1 overrides it.
    const bool split = (G == 16 || G == 32) && env_flag("RQMV_MOE_GLU_SPLIT", b.m == 1) && b.m <= kMoeOwnRouteMax;
    const int GL = split ? 2 * G : G;  // lanes per row pair in the launch
    const int total_rows = d.top * d.hidden + d.hidden_shared;
    const int rows_per_block = 4 * (64 / GL);
    int grid = (total_rows + rows_per_block - 1) / rows_per_block;
    const int cap = batch_grid_cap(cus, b.m);
    if (grid > cap) grid = cap;
    const size_t lds = stage_bytes_int(FMT, 1, nch);
    auto kernel = b.m > kMoeOwnRouteMax ? moe_glu_kernel<FMT, XF32, S, true>
                  : split                ? moe_glu_kernel<FMT, XF32, S, false, true>
                                         : moe_glu_kernel<FMT, XF32, S, false>;
    if (lds > 60000) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(kernel, dim3(grid, b.m), dim3(kMoeThreads), lds, stream, d, gate, up, gate_sh, up_sh, x, ws,
                       route_dense, GL, b);
    return hipGetLastError();
}

template <int FMT, bool XF32>
static hipError_t glu_slots(const MoeDims& d, const MoeBank& gate, const MoeBank& up, const MoeBank& gate_sh,
                            const MoeBank& up_sh, const void* x, MoeWorkspace ws, float* route_dense,
                            const MoeBatch& b, int cus, hipStream_t stream) {
    const int slots = (d.experts + 63) / 64;
#define RQ_GLU(S) glu_launch<FMT, XF32, S>(d, gate, up, gate_sh, up_sh, x, ws, route_dense, b, cus, stream)
    if (slots <= 1) return RQ_GLU(1);
    if (slots <= 2) return RQ_GLU(2);
    if (slots <= 4) return RQ_GLU(4);
    if (slots <= 8) return RQ_GLU(8);
    if (slots <= 16) return RQ_GLU(16);
    return RQ_GLU(32);
#undef RQ_GLU
}

template <int FMT>
static hipError_t glu_fmt(int xtype, const MoeDims& d, const MoeBank& gate, const MoeBank& up, const MoeBank& gate_sh,
                          const MoeBank& up_sh, const void* x, MoeWorkspace ws, float* route_dense,
                          const MoeBatch& b, int cus, hipStream_t stream) {
    if (d.experts > kTopkMaxExperts || d.top > 64 || d.top < 1) return hipErrorInvalidValue;
    if (xtype == 0) return glu_slots<FMT, true>(d, gate, up, gate_sh, up_sh, x, ws, route_dense, b, cus, stream);
    return glu_slots<FMT, false>(d, gate, up, gate_sh, up_sh, x, ws, route_dense, b, cus, stream);
}

hipError_t launch_moe_glu(int fmt, int xtype, const MoeDims& d, const MoeBank& gate, const MoeBank& up,
                          const MoeBank& gate_sh, const MoeBank& up_sh, const void* x, MoeWorkspace ws,
                          float* route_dense, const MoeBatch& b, int cus, hipStream_t stream) {
    switch (fmt) {
        case Q4_0: return glu_fmt<Q4_0>(xtype, d, gate, up, gate_sh, up_sh, x, ws, route_dense, b, cus, stream);
        case Q8_0: return glu_fmt<Q8_0>(xtype, d, gate, up, gate_sh, up_sh, x, ws, route_dense, b, cus, stream);
        case Q4_K: return glu_fmt<Q4_K>(xtype, d, gate, up, gate_sh, up_sh, x, ws, route_dense, b, cus, stream);
        case Q6_K: return glu_fmt<Q6_K>(xtype, d, gate, up, gate_sh, up_sh, x, ws, route_dense, b, cus, stream);
        default: return hipErrorInvalidValue;
    }
}

template <int FMT>
static hipError_t down_fmt(const MoeDims& d, const MoeBank& down, const MoeBank& down_sh, MoeWorkspace ws, float* y,
                           const MoeBatch& b, int cus, hipStream_t stream) {
    constexpr int CW = Traits<FMT>::CW;
    const int nch = (d.top * d.hidden + d.hidden_shared) / CW;
    // Lanes per output row (the order of each row's sum), at most 32. Every
    // workgroup stages the whole slot activation vector, so rows per
    // workgroup amortise it. The same at every batch size, so that a batch
    // stays bit-identical to one-position calls (16 lanes measured slower at
    // one position, 64 from two). RQMV_MOE_DOWN_G overrides it.
    const char* genv = getenv("RQMV_MOE_DOWN_G");
    int G = lanes_for(nch);
    if (G > 32) G = 32;
    if (genv && *genv) {
        const int g = atoi(genv);
        if (g == 8 || g == 16 || g == 32 || g == 64) G = g;
    }
    // At two positions 512-thread workgroups, from three 1024-thread ones,
    // each staging the slot activations once for more rows; at one position,
    // the split form below. Each row's sum is the same in every form, so
    // batches stay bit-identical to one-position calls. Measured on the
    // gguf_moe workload, us per step at 1 / 2 / 3 / 4 / 8 / 16 / 32 positions:
    // 256 threads 18.2 / 21.5 / 27.5 / 30.8 / 50.5 / 76.6 / 129.3, 512 threads
    // 18.4 / 20.3 / 27.2 / 29.2 / 48.3 / 75.0 / 127.7, the split form 17.1 /
    // 20.9; after cheaper staging, 512 against 1024 threads from two
    // positions: 19.8 / 26.7 / 28.6 / 47.0 / 73.7 / 126.6 against 21.1 / 25.9
    // / 27.8 / 46.0 / 73.3 / 126.5. 64 lanes per row (other sums) were faster
    // at one position only (17.0-17.3) and slower from two (21.1 / 29.0 / 33.6
    // / 50.6 / 79.0 / 135.3). RQMV_MOE_DOWN_WIDE=0/1 and RQMV_MOE_DOWN_THREADS
    // override the workgroup size, RQMV_MOE_DOWN_SPLIT=0/1 the split form (one
    // or two positions, 32 lanes).
    int threads = env_flag("RQMV_MOE_DOWN_WIDE", b.m >= 2) ? (b.m >= 3 ? 1024 : 512) : kMoeThreads;
    const char* tenv = getenv("RQMV_MOE_DOWN_THREADS");
    if (tenv && *tenv) {
        const int v = atoi(tenv);
        if (v == 256 || v == 512 || v == 1024) threads = v;
    }
    const int rows_per_block = threads / 64 * (64 / G);
    int grid = (d.d_model + rows_per_block - 1) / rows_per_block;
    const int cap = (batch_grid_cap(cus, b.m) * kMoeThreads + threads - 1) / threads;
    if (grid > cap) grid = cap;
    const size_t lds = stage_bytes_int(FMT, 1, nch);
    const bool ring = b.m > kMoeOwnRouteMax;
    auto kernel = ring ? (threads == 1024 ? moe_down_kernel<FMT, true, 1024>
                          : threads == 512 ? moe_down_kernel<FMT, true, 512>
                                           : moe_down_kernel<FMT, true>)
                       : (threads == 1024 ? moe_down_kernel<FMT, false, 1024>
                          : threads == 512 ? moe_down_kernel<FMT, false, 512>
                                           : moe_down_kernel<FMT, false>);
    // the split form: one row per wave on 512-thread workgroups
    if (!ring && G == 32 && env_flag("RQMV_MOE_DOWN_SPLIT", b.m == 1)) {
        threads = 512;
        grid = (d.d_model + threads / 64 - 1) / (threads / 64);
        const int scap = (batch_grid_cap(cus, b.m) * kMoeThreads + threads - 1) / threads;
        if (grid > scap) grid = scap;
        kernel = moe_down_kernel<FMT, false, 512, true>;
        // rows of 65-72 chunks (eight routed slots of 64-weight chunks and a
        // shared expert of the same width): a ninth wave per workgroup takes
        // the chunks past 64 of the eight rows, when one launch covers them.
        // On the gguf_moe workload (72 chunks) the step goes 17.18 -> 15.89 us
        // (graph replays, five alternating runs): no lane waits for a second
        // weight load after its first dot, and 576 threads stage the 576 items
        // in one round. RQMV_MOE_DOWN_TAIL=0 turns it off.
        const int tgrid = (d.d_model + 7) / 8;
        if (nch > 64 && nch <= 72 && tgrid <= (batch_grid_cap(cus, b.m) * kMoeThreads + 575) / 576 &&
            env_flag("RQMV_MOE_DOWN_TAIL", true)) {
            threads = 576;
            grid = tgrid;
            kernel = moe_down_kernel<FMT, false, 576, true, true>;
        }
    }
    if (lds > 65536) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(kernel, dim3(grid, b.m), dim3(threads), lds, stream, d, down, down_sh, ws, y, G, b);
    return hipGetLastError();
}

hipError_t launch_moe_down(int fmt, const MoeDims& d, const MoeBank& down, const MoeBank& down_sh, MoeWorkspace ws,
                           float* y, const MoeBatch& b, int cus, hipStream_t stream) {
    switch (fmt) {
        case Q4_0: return down_fmt<Q4_0>(d, down, down_sh, ws, y, b, cus, stream);
        case Q8_0: return down_fmt<Q8_0>(d, down, down_sh, ws, y, b, cus, stream);
        case Q4_K: return down_fmt<Q4_K>(d, down, down_sh, ws, y, b, cus, stream);
        case Q6_K: return down_fmt<Q6_K>(d, down, down_sh, ws, y, b, cus, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace rq
