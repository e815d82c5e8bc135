// Batch-1 and small-M (M <= 8; F16 weights M <= 16) dequant-dot matrix-vector
// kernels for gfx950.
//
// Work mapping. A wave's 64 lanes are split into 64/G groups of G lanes; a
// group owns R consecutive rows and its lanes take chunks g, g+G, g+2G, ...
// of those rows, so every load instruction of the wave reads contiguous 16-byte
// parts of a row (layout.h). Weights are read with buffer loads whose
// out-of-range form returns zeros without touching memory, so every lane
// issues the same loads and the waits stay exact. Each lane keeps R x M fp32
// partial sums; the G lanes of a group are reduced with DPP row operations (no
// atomics, no scratch) and the group's last lane writes the rows. Waves stride
// over row tiles, so a fixed, occupancy-sized grid covers any row count.
//
// Activations are staged once per workgroup into LDS as 16-bit integer digit
// words per 32-value block (stage.h), in a part-major layout ([m][part][chunk]
// 16-byte units) that makes the lanes' LDS reads conflict-free; the chunk
// products are exact int32 v_dot8_i32_i4 / v_dot4_i32_i8 sums scaled once per
// block (chunk.h).
//
// Reference counterparts: packed_lanes_body / packed_lanes4_body / packed_unit_dot
// (amd-nv-cpu.ll:2421-2664, 2674-3126, 2304-2364), where each lane of a wave
// takes one row, x is staged in LDS chunk by chunk and units are split over a
// team of waves.
#include <hip/hip_ext.h>
#include <stdlib.h>

#include "kernels.h"
#include "stage.h"

namespace rq {

// Walks this wave's (tile, step) pairs in order: step s of a tile takes chunk
// c = g + s*G of the tile's rows, for s < ceil(nch / G) on every lane (a lane
// whose chunk lies past the row does no work), so the whole wave reaches each
// tile's cross-lane reduction together. Tile and row indices are 32-bit (a
// weight has fewer than 2^31 rows, which its 4 GiB limit implies).
struct StepWalk {
    int tile, tiles, tile_stride, rows_per_wave;
    int s, steps, g, G, nch;
    __device__ bool valid() const { return tile < tiles; }
    __device__ int chunk() const { return g + s * G; }
    __device__ void next() {
        if (++s == steps) {
            s = 0;
            tile += tile_stride;
        }
    }
};

__device__ __forceinline__ StepWalk make_walk(const MvParams& p, int R, int g) {
    StepWalk w;
    (void)R;
    const int wpb = p.block >> 6, wave = threadIdx.x >> 6;
    w.rows_per_wave = p.rows_per_wave;
    w.tiles = p.tiles;
    // The wave's first tile: workgroup-major, or with p.spread (wide
    // workgroups whose tiles do not divide evenly over the waves) the first
    // four waves of every workgroup before the next four of any (waves w and
    // w + 4 share a SIMD), so that the last round's tiles spread over every CU
    // and SIMD instead of going to the first workgroups' waves, which at one
    // 512-thread workgroup per CU left half of the CUs with twice the last
    // round's work.
    if (p.spread && wpb > 4)
        w.tile = (wave & 3) + 4 * ((int)blockIdx.x + (int)gridDim.x * (wave >> 2));
    else
        w.tile = (int)blockIdx.x * wpb + wave;
    w.tile_stride = (int)gridDim.x * wpb;
    w.s = 0;
    w.steps = p.steps;
    w.g = g;
    w.G = p.G;
    w.nch = p.P.nch;
    return w;
}

// The walk's launch-shape constants (MvParams::g_shift .. steps) for G lanes
// per row and R rows per lane group.
static void set_walk(MvParams& p, int G, int R) {
    int sh = 0;
    while ((1 << sh) < G) ++sh;
    p.g_shift = sh;
    p.rows_per_wave = (64 >> sh) * R;
    p.tiles = (int)((p.rows + p.rows_per_wave - 1) / p.rows_per_wave);
    p.steps = (p.P.nch + G - 1) / G;
}

// Loads step `w` for the lane's R rows. Rows or chunks past the end (and the
// steps of a wave without a tile) load from a clamped in-range address
// instead; their results are never added.
template <int FMT, int R>
__device__ __forceinline__ void load_rows(const MvParams& p, const StepWalk& w, int sub, ChunkData<FMT> (&d)[R]) {
    const int tile = w.tile < w.tiles ? w.tile : w.tiles - 1;
    const int row0 = tile * w.rows_per_wave + sub * R, rows = (int)p.rows;
    const int c = w.chunk() < w.nch ? w.chunk() : w.nch - 1;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int row = row0 + r < rows ? row0 + r : rows - 1;
        if constexpr (FMT == F16) {
            const bool second = row >= p.split;
            Planes P = p.P;
            P.base = second ? p.P2.base : p.P.base;
            load_chunk<FMT>(P, second ? row - p.split : row, c, d[r]);
        } else {
            load_chunk<FMT>(p.P, row, c, d[r]);
        }
    }
}

// The tile's cross-lane sums and its epilogue (MvParams::epi; the GLU
// epilogue runs with M = 1 and an even R, so that a lane group holds each
// (gate, up) row pair). NORM: the rmsnorm factor multiplies the sums first.
template <int M, int R, bool NORM = false>
__device__ __forceinline__ void finish_tile(const MvParams& p, int row0, int g, float (&acc)[R][M],
                                            float norm_scale = 1.f) {
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int mm = 0; mm < M; ++mm) {
            acc[r][mm] = group_sum(acc[r][mm], p.G);
            if constexpr (NORM) acc[r][mm] *= norm_scale;
        }
    if (g == p.G - 1) {
        if (p.epi == kEpiPlain) {
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (row0 + r < (int)p.rows)
#pragma unroll
                    for (int mm = 0; mm < M; ++mm) p.y[(int64_t)mm * p.ldy + row0 + r] = acc[r][mm];
        } else {
            // silu(gate) * up, silu(v) = v * sigmoid(v), sigmoid = 0.5 (tanh(v / 2) + 1) (recipe.rs:22662-22668)
#pragma unroll
            for (int r = 0; r + 1 < R; r += 2)
                if (row0 + r + 1 < (int)p.rows) {
                    const float gt = acc[r][0];
                    p.y[(row0 + r) / 2] = gt * (0.5f * (tanhf(0.5f * gt) + 1.0f)) * acc[r + 1][0];
                }
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int mm = 0; mm < M; ++mm) acc[r][mm] = 0.f;
}

// load_rows through the weight's buffer resource: lanes whose row, chunk or
// tile lies past the end (and every lane of a step past the wave's last)
// load nothing and get zeros.
template <int FMT, int R>
__device__ __forceinline__ void load_rows_rs(const MvParams& p, __amdgpu_buffer_rsrc_t rs, const StepWalk& w, int sub,
                                             ChunkData<FMT> (&d)[R]) {
    const bool live = w.tile < w.tiles && w.chunk() < w.nch;
    const int row0 = w.tile * w.rows_per_wave + sub * R, rows = (int)p.rows;
#pragma unroll
    for (int r = 0; r < R; ++r) load_chunk_rs<FMT>(rs, p.P, (uint32_t)(row0 + r), w.chunk(), live && row0 + r < rows, d[r]);
}

// One step of matvec_int: the lane's chunk of its R rows against the staged
// digits of every activation row; the tile's reduction after its last step.
template <int FMT, int M, int R, bool NORM = false, bool FIN = true>
__device__ __forceinline__ void step_int(const MvParams& p, const StepWalk& w, int sub, int g, const ChunkData<FMT> (&d)[R],
                                         float (&acc)[R][M], const uint4* xd, const uint4* xb, bool outliers,
                                         float norm_scale = 1.f) {
    constexpr int XP = Traits<FMT>::XP, XR = Traits<FMT>::XR;
    const int nch = p.P.nch;
    const int c = w.chunk();
    const int row0 = w.tile * w.rows_per_wave + sub * R, rows = (int)p.rows;
    if (c < nch) {
        ChunkWords<FMT> cw[R];
#pragma unroll
        for (int r = 0; r < R; ++r) chunk_words<FMT>(d[r], cw[r]);
        // one activation row's digits live at a time; the weights stay in registers
#pragma unroll
        for (int mm = 0; mm < M; ++mm) {
            uint4 xv[XP];
            uint4 bv[2];
#pragma unroll
            for (int j = 0; j < XP; ++j) xv[j] = xd[(mm * XP + j) * nch + c];
            bv[0] = xb[(mm * XR + 0) * nch + c];
            bv[1] = xb[(mm * XR + 1) * nch + c];
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (row0 + r < rows) dot_int_w<FMT>(d[r], cw[r], c, xv, bv, acc[r][mm]);
            if (__builtin_expect(outliers && wave_has_outlier(bv[0]), 0)) {
#pragma unroll
                for (int r = 0; r < R; ++r)
                    if (row0 + r < rows) dot_outliers<FMT>(d[r], c, xb + mm * XR * nch + c, nch, acc[r][mm]);
            }
        }
    }
    if (FIN && w.s == w.steps - 1) finish_tile<M, R, NORM>(p, row0, g, acc, norm_scale);
}

// Quantized weights, integer dot of staged activation digits (chunk.h,
// stage.h). A ring of NB register buffers: while one step is computed, the
// loads of the next NB - 1 are in flight, and the buffer just computed is
// refilled for the step NB ahead. All NB first steps' weight loads are issued
// before the activations are staged, so the staging overlaps them. NORM: the
// rmsnorm prologue (M = 1, fp32 activations).
template <int M, int R>
constexpr int ring_depth() {
    return 2;  // deeper rings (3, 4) measured slower on gfx950 at batch 1
}

template <int FMT, int M, int R, bool XF32, bool NORM = false>
__global__ void __launch_bounds__(512) matvec_int(MvParams p) {
    constexpr int XP = Traits<FMT>::XP;
    constexpr int NB = ring_depth<M, R>();
    extern __shared__ uint4 smem[];
    __shared__ float block_scalar[8];  // NORM: the waves' sums of squares
    __shared__ int wave_flags[8];      // the waves' "a staged block holds an outlier"
    const int nch = p.P.nch;
    uint4* xd = smem;
    uint4* xb = smem + M * XP * nch;
    const int lane = threadIdx.x & 63, g = lane & (p.G - 1), sub = lane >> p.g_shift;
    const __amdgpu_buffer_rsrc_t rs = planes_rsrc(p.P);
    StepWalk w[NB];
    w[0] = make_walk(p, R, g);
#pragma unroll
    for (int i = 1; i < NB; ++i) {
        w[i] = w[i - 1];
        w[i].next();
    }

    ChunkData<FMT> buf[NB][R];
    NormIn nin{};
    float ssq = 0.f;  // NORM: this thread's share of sum (x + delta)^2
    if constexpr (NORM) nin = NormIn{p.norm_w, p.delta, blockIdx.x == 0 ? p.x_out : nullptr};
    if (stage_items<FMT>(nch, M) <= kStageNJ * p.block) {
        StageItem<XF32, NORM> it[kStageNJ];
        stage_multi_issue<FMT, XF32, NORM>(nch, p.K, p.x, p.ldx, M, p.block, it, nin);
        // keep the activation loads ahead of the weight loads: waiting for them
        // then leaves the weight loads in flight
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("" ::: "memory");
#pragma unroll
        for (int i = 0; i < NB; ++i) load_rows_rs<FMT, R>(p, rs, w[i], sub, buf[i]);
        publish_outliers(
            stage_multi_finish<FMT, XF32, NORM>(nch, p.K, M, p.block, it, xd, reinterpret_cast<float*>(xb), nin, &ssq),
            wave_flags);
    } else {
#pragma unroll
        for (int i = 0; i < NB; ++i) load_rows_rs<FMT, R>(p, rs, w[i], sub, buf[i]);
        publish_outliers(
            stage_all<FMT, XF32, NORM>(nch, p.K, p.x, p.ldx, M, p.block, xd, reinterpret_cast<float*>(xb), nin, &ssq),
            wave_flags);
    }
    if constexpr (NORM) {
        ssq = group_sum(ssq, 64);
        if (lane == 63) block_scalar[threadIdx.x >> 6] = ssq;
    }
    __syncthreads();
    const bool outliers = read_outliers(wave_flags, p.block);
    float norm_scale = 1.f;
    if constexpr (NORM) {  // the waves' sums in order: every workgroup forms the same factor
        float t = 0.f;
        for (int i = 0; i < (p.block >> 6); ++i) t += block_scalar[i];
        norm_scale = 1.0f / sqrtf(t / (float)p.K + p.eps);
    }

    float acc[R][M];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int mm = 0; mm < M; ++mm) acc[r][mm] = 0.f;
    for (;;) {
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            if (!w[i].valid()) goto done;
            step_int<FMT, M, R, NORM>(p, w[i], sub, g, buf[i], acc, xd, xb, outliers, norm_scale);
            // this buffer takes the step after the latest one issued
            w[i] = w[(i + NB - 1) % NB];
            w[i].next();
            load_rows_rs<FMT, R>(p, rs, w[i], sub, buf[i]);
        }
    }
done:
    return;
}

// Two waves per row tile (k2_shape; M = 1 or 2 activation rows): each row
// tile taken by two waves of one workgroup, one per half of the tile's steps
// (steps [0, ceil(S / 2)) and the rest), the first half's waves in the
// workgroup's first half. The workgroup
// stages x once for twice the waves, so each thread encodes half the items of
// the one-wave form before the first dot, and each wave walks half the steps.
// A wave takes up to kK2MaxTiles tiles (striding like matvec_int); at the end
// of each tile it writes its rows' group sums to LDS, and after the one
// barrier each row is written as half 0 + half 1. NORM: the rmsnorm prologue
// (M = 1, fp32 activations), its factor applied to each row's sum; with the
// GLU epilogue (kEpiGlu, M = 1) a tile's two rows are a (gate, up) pair and
// the pair writes silu(gate) * up.
constexpr int kK2MaxTiles = 8;
template <int FMT, int R, bool XF32 = false, int M = 1, bool NORM = false>
__global__ void __launch_bounds__(1024) matvec_int_k2(MvParams p) {
    constexpr int NB = 2;
    constexpr int XP = Traits<FMT>::XP;
    extern __shared__ uint4 smem[];
    __shared__ int wave_flags[16];
    __shared__ float block_scalar[16];  // NORM: the waves' sums of squares
    __shared__ float part[2][8][kK2MaxTiles][8 * M];  // [half][row wave][tile of the wave][row of the tile, x row]
    const int nch = p.P.nch;
    uint4* xd = smem;
    uint4* xb = smem + M * XP * nch;
    const int lane = threadIdx.x & 63, g = lane & (p.G - 1), sub = lane >> p.g_shift;
    const int wave = threadIdx.x >> 6, half = p.block >> 7;  // row waves per workgroup
    const int kh = wave >= half ? 1 : 0, rw = wave - kh * half;
    const __amdgpu_buffer_rsrc_t rs = planes_rsrc(p.P);
    const int s_mid = (p.steps + 1) >> 1;
    StepWalk w[NB];
    w[0].rows_per_wave = p.rows_per_wave;
    w[0].tiles = p.tiles;
    w[0].tile = (int)blockIdx.x * half + rw;
    w[0].tile_stride = (int)gridDim.x * half;
    w[0].s = kh ? s_mid : 0;
    w[0].steps = kh ? p.steps : s_mid;
    w[0].g = g;
    w[0].G = p.G;
    w[0].nch = nch;
    w[1] = w[0];
    w[1].next();
    if (kh) w[1].s = w[1].s == 0 ? s_mid : w[1].s;  // (a new tile starts the second half at its midpoint)
    ChunkData<FMT> buf[NB][R];
    NormIn nin{};
    float ssq = 0.f;  // NORM: this thread's share of sum (x + delta)^2
    if constexpr (NORM) nin = NormIn{p.norm_w, p.delta, blockIdx.x == 0 ? p.x_out : nullptr};
    constexpr int NJ = NORM ? kStageNJNorm : kStageNJ;
    StageItem<XF32, NORM> it[NJ];
    stage_multi_issue<FMT, XF32, NORM, NJ>(nch, p.K, p.x, p.ldx, M, p.block, it, nin);
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
#pragma unroll
    for (int i = 0; i < NB; ++i) load_rows_rs<FMT, R>(p, rs, w[i], sub, buf[i]);
    publish_outliers(stage_multi_finish<FMT, XF32, NORM, NJ>(nch, p.K, M, p.block, it, xd, reinterpret_cast<float*>(xb),
                                                             nin, &ssq),
                     wave_flags);
    if constexpr (NORM) {
        ssq = group_sum(ssq, 64);
        if (lane == 63) block_scalar[wave] = ssq;
    }
    __syncthreads();
    const bool outliers = read_outliers(wave_flags, p.block);
    float norm_scale = 1.f;
    if constexpr (NORM) {  // the waves' sums in order: every workgroup forms the same factor
        float t = 0.f;
        for (int i = 0; i < (p.block >> 6); ++i) t += block_scalar[i];
        norm_scale = 1.0f / sqrtf(t / (float)p.K + p.eps);
    }
    float acc[R][M];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int mm = 0; mm < M; ++mm) acc[r][mm] = 0.f;
    int j = 0;  // the wave's finished tiles
    for (;;) {
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            if (!w[i].valid()) goto done;
            step_int<FMT, M, R, false, false>(p, w[i], sub, g, buf[i], acc, xd, xb, outliers);
            if (w[i].s == w[i].steps - 1) {  // the tile's last step of this half
#pragma unroll
                for (int r = 0; r < R; ++r)
#pragma unroll
                    for (int mm = 0; mm < M; ++mm) {
                        const float t = group_sum(acc[r][mm], p.G);
                        if (g == p.G - 1) part[kh][rw][j][(sub * R + r) * M + mm] = t;
                        acc[r][mm] = 0.f;
                    }
                ++j;
            }
            w[i] = w[(i + NB - 1) % NB];
            w[i].next();
            if (kh && w[i].s == 0) w[i].s = s_mid;
            load_rows_rs<FMT, R>(p, rs, w[i], sub, buf[i]);
        }
    }
done:
    __syncthreads();
    const int rpw = p.rows_per_wave, per_wg = half * kK2MaxTiles * rpw;
    const bool glu = p.epi == kEpiGlu;
    for (int e = threadIdx.x; e < per_wg; e += p.block) {
        const int k = e % rpw, jj = (e / rpw) % kK2MaxTiles, r_w = e / (rpw * kK2MaxTiles);
        const int tile = (int)blockIdx.x * half + r_w + jj * (int)gridDim.x * half;
        const int row = tile * rpw + k;
        if (tile >= p.tiles || row >= (int)p.rows) continue;
        if (glu) {  // (M = 1) the pair's even row writes silu(gate) * up (recipe.rs:22662-22668, as finish_tile)
            if ((k & 1) == 0 && row + 1 < (int)p.rows) {
                float gt = part[0][r_w][jj][k] + part[1][r_w][jj][k];
                float up = part[0][r_w][jj][k + 1] + part[1][r_w][jj][k + 1];
                if constexpr (NORM) {
                    gt *= norm_scale;
                    up *= norm_scale;
                }
                p.y[row / 2] = gt * (0.5f * (tanhf(0.5f * gt) + 1.0f)) * up;
            }
            continue;
        }
#pragma unroll
        for (int mm = 0; mm < M; ++mm) {
            float v = part[0][r_w][jj][k * M + mm] + part[1][r_w][jj][k * M + mm];
            if constexpr (NORM) v *= norm_scale;
            p.y[(int64_t)mm * p.ldy + row] = v;
        }
    }
}

// Burst form of matvec_int for long rows at one or two activation rows: every
// wave owns U units (row, step) fixed at launch and issues the loads of all of
// them before anything else, so that the whole matrix is requested within the
// first moments of the launch and HBM streams it at full rate; then the
// activations are staged (their loads were issued first, so waiting for them
// leaves every weight load in flight), and the units are computed in the order
// their loads return. Rows are dealt to waves round-robin (row = wave + r *
// waves), so that the waves' r-th rows together are one contiguous region.
// A wave covers a row with all 64 lanes (chunk lane + 64 s at step s); S
// steps per row, U / S rows per wave.
template <int FMT, int M, int U, bool XF32>
__global__ void __launch_bounds__(256) matvec_burst(MvParams p, int S) {
    constexpr int XP = Traits<FMT>::XP, XR = Traits<FMT>::XR;
    extern __shared__ uint4 smem[];
    const int nch = p.P.nch;
    uint4* xd = smem;
    uint4* xb = smem + M * XP * nch;
    const int lane = threadIdx.x & 63;
    const int waves = (int)gridDim.x * (p.block >> 6);
    const int wave = (int)blockIdx.x * (p.block >> 6) + (int)(threadIdx.x >> 6);
    const __amdgpu_buffer_rsrc_t rs = planes_rsrc(p.P);
    const int rows = (int)p.rows;

    __shared__ int wave_flags[4];
    ChunkData<FMT> d[U];
    StageItem<XF32> it[kStageNJ];
    stage_multi_issue<FMT, XF32>(nch, p.K, p.x, p.ldx, M, p.block, it);
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int r = u / S, st = u - r * S;
        const int row = wave + r * waves, c = lane + 64 * st;
        load_chunk_rs<FMT>(rs, p.P, (uint32_t)row, c, row < rows && c < nch, d[u]);
    }
    publish_outliers(stage_multi_finish<FMT, XF32>(nch, p.K, M, p.block, it, xd, reinterpret_cast<float*>(xb)),
                     wave_flags);
    __syncthreads();
    const bool outliers = read_outliers(wave_flags, p.block);

    float acc[M];
#pragma unroll
    for (int mm = 0; mm < M; ++mm) acc[mm] = 0.f;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int r = u / S, st = u - r * S;
        const int row = wave + r * waves, c = lane + 64 * st;
        if (c < nch) {
            ChunkWords<FMT> cw;
            chunk_words<FMT>(d[u], cw);
#pragma unroll
            for (int mm = 0; mm < M; ++mm) {
                uint4 xv[XP];
                uint4 bv[2];
#pragma unroll
                for (int j = 0; j < XP; ++j) xv[j] = xd[(mm * XP + j) * nch + c];
                bv[0] = xb[(mm * XR + 0) * nch + c];
                bv[1] = xb[(mm * XR + 1) * nch + c];
                dot_int_w<FMT>(d[u], cw, c, xv, bv, acc[mm]);
                if (__builtin_expect(outliers && wave_has_outlier(bv[0]), 0))
                    dot_outliers<FMT>(d[u], c, xb + mm * XR * nch + c, nch, acc[mm]);
            }
        }
        if (st == S - 1) {
#pragma unroll
            for (int mm = 0; mm < M; ++mm) {
                const float v = group_sum(acc[mm], 64);
                if (lane == 63 && row < rows) p.y[(int64_t)mm * p.ldy + row] = v;
                acc[mm] = 0.f;
            }
        }
    }
}

// F16 weights (router-sized): fp16 activations through v_dot2_f32_f16, fp32
// activations through exact fp32 fma.
template <int M, int R, bool XF32>
__global__ void __launch_bounds__(512) matvec_f16w(MvParams p) {
    extern __shared__ uint4 smem[];
    const int nch = p.P.nch;
    const int lane = threadIdx.x & 63, g = lane & (p.G - 1), sub = lane >> p.g_shift;
    StepWalk w = make_walk(p, R, g);
    ChunkData<F16> cur[R];
    load_rows<F16, R>(p, w, sub, cur);
    if constexpr (XF32)
        stage_f32_quads(nch, p.K, p.x, p.ldx, M, p.block, reinterpret_cast<float4*>(smem));
    else
        stage_f16_pairs(nch, p.K, p.x, p.ldx, M, p.block, smem);
    __syncthreads();

    float acc[R][M];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int mm = 0; mm < M; ++mm) acc[r][mm] = 0.f;
    bool loaded = true;
    while (w.valid()) {
        if (!loaded) load_rows<F16, R>(p, w, sub, cur);
        loaded = false;
        const int c = w.chunk();
        const int row0 = w.tile * w.rows_per_wave + sub * R, rows = (int)p.rows;
        if (c < nch) {
            if constexpr (XF32) {
#pragma unroll
                for (int r = 0; r < R; ++r)
                    if (row0 + r < rows)
#pragma unroll
                        for (int mm = 0; mm < M; ++mm)
                            acc[r][mm] += chunk_dot_f32(cur[r], reinterpret_cast<const float4*>(smem), nch, c, mm);
            } else if constexpr (M <= 8) {
                uint4 xv[M][8];
#pragma unroll
                for (int mm = 0; mm < M; ++mm)
#pragma unroll
                    for (int j = 0; j < 8; ++j) xv[mm][j] = smem[(mm * 8 + j) * nch + c];
#pragma unroll
                for (int r = 0; r < R; ++r)
                    if (row0 + r < rows) dot_f16w<M>(cur[r], xv, acc[r]);
            } else {
                // one activation row's pieces at a time (all of them would not
                // fit in registers); each sum sees the same operations in the
                // same order as at any other M
#pragma unroll
                for (int mm = 0; mm < M; ++mm) {
                    uint4 xv[1][8];
#pragma unroll
                    for (int j = 0; j < 8; ++j) xv[0][j] = smem[(mm * 8 + j) * nch + c];
#pragma unroll
                    for (int r = 0; r < R; ++r)
                        if (row0 + r < rows) dot_f16w<1>(cur[r], xv, &acc[r][mm]);
                }
            }
        }
        if (w.s == w.steps - 1) finish_tile<M, R>(p, row0, g, acc);
        w.next();
    }
}

template <int FMT>
__global__ void __launch_bounds__(256) dequant_kernel(Planes P, int64_t rows, int cols, float* out) {
    constexpr int CW = Traits<FMT>::CW;
    const int64_t total = rows * P.nch;
    for (int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; u < total; u += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = u / P.nch;
        const int c = (int)(u % P.nch);
        ChunkData<FMT> d;
        load_chunk<FMT>(P, row, c, d);
        float w[CW];
        decode_chunk<FMT>(d, c, w);
        float* o = out + row * cols + (int64_t)c * CW;
        const int valid = cols - c * CW < CW ? cols - c * CW : CW;
#pragma unroll
        for (int v = 0; v < CW; ++v)
            if (v < valid) o[v] = w[v];
    }
}

size_t matvec_lds_bytes(int fmt, int xtype, int M, int cols) {
    if (!format_info(fmt).chunk_values) return 0;
    const int nch = (int)chunks_per_row(fmt, cols);
    if (fmt == F16) return stage_bytes_f16w(xtype == X_F32, M, nch);
    return stage_bytes_int(fmt, M, nch);
}

static int env_int(const char* name, int fallback) {
    const char* v = getenv(name);
    return v && *v ? atoi(v) : fallback;
}

// Two waves per row tile (matvec_int_k2), at one or two activation rows, 32 lanes
// and one row per lane group (two rows per tile), each wave taking half of a
// tile's steps:
// - long rows: Q4_K and Q4_0 rows of more than 128 chunks, up to 4,096 rows,
//   one tile per wave on at most one 1,024-thread workgroup per CU. Measured
//   (kernel us, three alternating runs): with fp16 x, Q4_K 14336->4096 10.37
//   (64 lanes, two rows per group) -> 10.00 (32 lanes, one row) -> 9.07-9.38
//   (two waves per tile); Q4_0 9.78 -> 9.94 -> 8.82, where two waves per tile
//   at 64 lanes and two rows measured slower (10.44). With fp32 x (the decode
//   step's down product, through the fused entry point) 32 lanes and one row
//   alone were slower (568 -> 548 tok/s) and two waves per tile faster (597.0
//   -> 614.1).
// - rows of 64-128 chunks (Q8_0: 64-192 chunks of 32 weights) on two
//   512-thread workgroups per CU, each wave taking up to kK2MaxTiles tiles,
//   when every wave has a tile. With fp16 x: Q4_K 4096->14336 9.33 -> 8.63
//   us, Q6_K 5120->25600 22.64 -> 20.69, Q4_0 4096->14336 8.55 -> 8.47, Q8_0
//   5120x5120 8.39 -> 7.41 (three alternating runs; 384, 448 and 640
//   workgroups and one 1,024-thread workgroup per CU were slower); with fp32
//   x, Q8_0 4096x4096 6.40 -> 6.20 (6.36 in the burst form) and the decode
//   step's output product (through the fused entry point) 607.1 -> 614.1
//   tok/s.
// Both at one or two activation rows: at two, Q6_K 5120->25600 35.64 -> 32.36
// us, Q8_0 5120x5120 10.58 -> 9.51.
// RQMV_K2=0 turns both off, RQMV_K2_SHORT=0 the second.
static bool k2_shape(int fmt, int64_t rows, int64_t nch, int M, int xtype, int cus, LaunchShape& s) {
    // (three and four activation rows of Q8_0 and three of Q6_K, where it beats
    // the matrix-core forms: Q6_K 5120->25600 at three rows 38.8 -> 33.6 us, at
    // four a tie, 39.6 against 38.9)
    if (M > (fmt == Q8_0 ? 4 : fmt == Q6_K ? 3 : 2) || !env_int("RQMV_K2", 1)) return false;
    const int64_t tiles = (rows + 1) / 2;
    if ((fmt == Q4_K || fmt == Q4_0) && nch > 128) {
        if (tiles > (int64_t)8 * cus) return false;
        s.block = 1024;
        s.grid = (int)((tiles + 7) / 8);
    } else if (fmt != F16 && nch >= 64 && nch <= (fmt == Q8_0 ? 192 : 128) && env_int("RQMV_K2_SHORT", 1)) {
        // two 512-thread workgroups per CU, or one of 1,024 threads where x
        // needs more than four items per thread of 512, or where one row of
        // fp32 activations leaves one tile per wave pair (each CU then stages the
        // heavier fp32 row once, not twice: Q8_0 4096x4096 6.16 -> 5.97 us,
        // the decode step, whose 4096x4096 output projection this is, 621.4
        // -> 625.8 tok/s; with fp16 x, or more tiles per pair, it measured
        // slower: Q4_K 4096->14336 8.36 -> 8.96 us median, Q8_0 5120x5120
        // 7.1 -> 7.8, the decode step with every fp32 product wide 614.0)
        const bool fp32_one_tile = xtype == X_F32 && M == 1 && tiles <= (int64_t)2 * cus * 4;
        s.block = (int64_t)stage_items_host(fmt, nch, M) > (int64_t)kStageNJ * 512 || fp32_one_tile ? 1024 : 512;
        s.grid = s.block == 1024 ? cus : 2 * cus;
        const int64_t stride = (int64_t)s.grid * (s.block / 128);
        if (tiles < stride || (tiles + stride - 1) / stride > kK2MaxTiles) return false;
    } else {
        return false;
    }
    // (the kernel stages x in one pass of at most kStageNJ items per thread)
    if ((int64_t)stage_items_host(fmt, nch, M) > (int64_t)kStageNJ * s.block) return false;
    s.G = 32;
    s.R = 1;
    s.k2 = true;
    return true;
}

static LaunchShape plan_matvec_impl(int fmt, int64_t rows, int64_t cols, int M, int xtype, int cus, bool k2) {
    LaunchShape s;
    const int64_t nch = chunks_per_row(fmt, cols);
    if (k2 && k2_shape(fmt, rows, nch, M, xtype, cus, s)) return s;
    int G = 64;
    while (G > 8 && G > nch) G >>= 1;
    // Q6_K rows of 65-95 chunks (5120 columns: 80) leave a 64-lane group's
    // second step three-quarters idle, and Q6_K's chunks are the costliest to
    // decode: 32 lanes per row measured faster (Q6_K 5120->25600 27.6 -> 24.5
    // us; Q4_K at 5120 columns a tie; Q6_K at 3584, 4096 and 14336 columns
    // faster at 64: 14.9 / 13.5 / 15.0 against 14.7 / 14.0 / 17.4).
    if (fmt == Q6_K && G == 64 && nch > 64 && nch < 96) G = 32;
    s.G = G;
    s.R = M <= 2 ? 2 : 1;
    if (xtype == X_F32) s.R = M == 1 ? 2 : 1;
    // Q8_0 chunks are 32 weights (two steps per lane of a 64-chunk row): one
    // row per lane group measured faster at M = 1 and 2 (4096^2 fp32 x median
    // 6.3 -> 5.7 us); the other formats measured faster with two
    if (fmt == Q8_0) s.R = 1;
    // Long rows stage a large activation slice per block: fewer, wider blocks
    // amortise it. Short rows favour more resident blocks per CU.
    const bool long_rows = nch > 128;
    s.block = long_rows ? 512 : 256;
    int per_cu = long_rows ? 1 : 2;
    // Long Q4_K rows at one fp16 activation row (where the long-row form does
    // not apply): 32 lanes per row and one row per lane group (Q4_K
    // 14336->4096 kernel 10.37 -> 10.00 us with 64 lanes and two rows before
    // it; with fp32 rows it was slower, 568 -> 548 tok/s on the decode step).
    if (fmt == Q4_K && M == 1 && long_rows && xtype == X_F16) {
        s.G = 32;
        s.R = 1;
    }
    // Small products at one or two activation rows, whose tiles would not give
    // every CU a workgroup, spread them over smaller workgroups of one row per
    // lane group (the MoE router, 257 x 2048 F16: 17 -> 65 workgroups; the MoE
    // step 19.7 -> 18.9 us). With 16 rows the smaller workgroups stage x twice as often and
    // the batched router measured slower (MoE step at 16 positions 82.4 -> 85.0 us).
    if (M <= 2 && ((rows + (64 / G) * s.R - 1) / ((64 / G) * s.R) + s.block / 64 - 1) / (s.block / 64) < cus) {
        s.R = 1;
        s.block = 128;
    }
    // tuning overrides, taken only within what the kernels are built for
    // (lanes per row a power of two from 8 to 64; workgroups of whole waves
    // up to the kernels' launch bound of 512 threads)
    const int env_g = env_int("RQMV_G", s.G), env_r = env_int("RQMV_R", s.R), env_b = env_int("RQMV_BLOCK", s.block);
    if (env_g == 8 || env_g == 16 || env_g == 32 || env_g == 64) s.G = env_g;
    if (env_r == 1 || env_r == 2 || env_r == 4) s.R = env_r;
    if (env_b >= 64 && env_b <= 512 && env_b % 64 == 0) s.block = env_b;
    const int64_t rows_per_wave = (int64_t)(64 / s.G) * s.R;
    const int64_t tiles = (rows + rows_per_wave - 1) / rows_per_wave;
    const int wpb = s.block / 64;
    int64_t grid = (tiles + wpb - 1) / wpb;
    const int per_cu_env = env_int("RQMV_BLOCKS_PER_CU", per_cu);
    const int64_t cap = (int64_t)cus * (per_cu_env >= 1 ? per_cu_env : per_cu);
    if (grid > cap) grid = cap;
    s.grid = env_int("RQMV_GRID", (int)grid);
    if (s.grid < 1) s.grid = 1;
    return s;
}

bool k2_takes(int fmt, int64_t rows, int64_t cols, int M, int xtype, int cus) {
    LaunchShape s;
    return k2_shape(fmt, rows, chunks_per_row(fmt, cols), M, xtype, cus, s);
}

LaunchShape plan_matvec(int fmt, int64_t rows, int64_t cols, int M, int xtype, int cus) {
    return plan_matvec_impl(fmt, rows, cols, M, xtype, cus, true);
}

template <typename K>
static hipError_t launch_kernel(K kernel, const MvParams& p_in, const LaunchShape& s, size_t lds, hipStream_t stream,
                                hipEvent_t ev0, hipEvent_t ev1) {
    MvParams p = p_in;
    p.block = s.block;
    p.G = s.G;
    set_walk(p, s.G, s.R);
    if (lds > 65536) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)lds);
        if (e != hipSuccess) return e;
    }
    if (ev0 || ev1)  // events recorded by the dispatch itself: its start and completion
        hipExtLaunchKernelGGL(kernel, dim3(s.grid), dim3(s.block), (uint32_t)lds, stream, ev0, ev1, 0u, p);
    else
        hipLaunchKernelGGL(kernel, dim3(s.grid), dim3(s.block), lds, stream, p);
    return hipGetLastError();
}

template <int FMT, int M, int R>
static hipError_t launch_one(int xtype, const MvParams& p, const LaunchShape& s, hipStream_t stream, hipEvent_t ev0,
                             hipEvent_t ev1) {
    const size_t lds = matvec_lds_bytes(FMT, xtype, M, p.K);
    if constexpr (FMT == F16) {
        if (xtype == X_F16) return launch_kernel(matvec_f16w<M, R, false>, p, s, lds, stream, ev0, ev1);
        return launch_kernel(matvec_f16w<M, R, true>, p, s, lds, stream, ev0, ev1);
    } else {
        if (s.k2) {  // two waves per row tile (k2_shape)
            if constexpr ((M <= 2 || ((M == 3 || M == 4) && FMT == Q8_0) || (M == 3 && FMT == Q6_K)) && R == 1) {
                if (xtype == X_F16) return launch_kernel(matvec_int_k2<FMT, 1, false, M>, p, s, lds, stream, ev0, ev1);
                return launch_kernel(matvec_int_k2<FMT, 1, true, M>, p, s, lds, stream, ev0, ev1);
            }
            return hipErrorInvalidValue;
        }
        if constexpr (M == 3) {
            return hipErrorInvalidValue;  // (three rows run in the split form only)
        } else {
            if (xtype == X_F16) return launch_kernel(matvec_int<FMT, M, R, false>, p, s, lds, stream, ev0, ev1);
            return launch_kernel(matvec_int<FMT, M, R, true>, p, s, lds, stream, ev0, ev1);
        }
    }
}

template <int FMT>
static hipError_t launch_fmt(int xtype, int M, const MvParams& p, const LaunchShape& s, hipStream_t stream,
                             hipEvent_t ev0, hipEvent_t ev1) {
    switch (M * 16 + s.R) {
        case 16 + 1: return launch_one<FMT, 1, 1>(xtype, p, s, stream, ev0, ev1);
        case 16 + 2: return launch_one<FMT, 1, 2>(xtype, p, s, stream, ev0, ev1);
        case 16 + 4: return launch_one<FMT, 1, 4>(xtype, p, s, stream, ev0, ev1);
        case 32 + 1: return launch_one<FMT, 2, 1>(xtype, p, s, stream, ev0, ev1);
        case 32 + 2: return launch_one<FMT, 2, 2>(xtype, p, s, stream, ev0, ev1);
        case 48 + 1:  // three rows: Q8_0 and Q6_K in the split form only
            if constexpr (FMT == Q8_0 || FMT == Q6_K) return launch_one<FMT, 3, 1>(xtype, p, s, stream, ev0, ev1);
            return hipErrorInvalidValue;
        case 64 + 1: return launch_one<FMT, 4, 1>(xtype, p, s, stream, ev0, ev1);
        case 128 + 1: return launch_one<FMT, 8, 1>(xtype, p, s, stream, ev0, ev1);
        case 256 + 1:  // sixteen activation rows: F16 weights only (a router over a batch)
            if constexpr (FMT == F16) return launch_one<FMT, 16, 1>(xtype, p, s, stream, ev0, ev1);
            return hipErrorInvalidValue;
        default: return hipErrorInvalidValue;
    }
}

// When the burst form runs, and its units per wave. Measured on MI355X (one
// product, weights rotating through HBM): it wins on products of a few tens of
// MB at most, whose ring form holds one tile per wave anyway (Q4_K 4096x4096,
// fp16 x: 6.03 -> 5.21 us; Q8_0 4096x4096, fp32 x: 6.27 -> 5.68 us, each at
// U = 4), and loses on larger ones, where all of a wave's loads in flight at
// once delay its first row and the tail (Q4_K 4096->14336: 9.5 -> 10.7 us at
// U = 4, 11.3-12.4 at U = 2, 6, 8). U = 4 units: 4 rows of one step, or 2 of
// two. RQMV_BURST=0 turns it off, RQMV_BURST_U forces U.
constexpr int64_t kBurstMaxBytes = 20ll << 20;

static bool burst_plan(int fmt, int64_t rows, int64_t nch, int64_t row_bytes, int M, int& U, int& S, int& grid) {
    if (env_int("RQMV_BURST", 1) == 0 || M > 2 || fmt == F16 || nch < 48) return false;
    if (rows * row_bytes > kBurstMaxBytes && env_int("RQMV_BURST_U", 0) == 0) return false;
    S = (int)((nch + 63) / 64);
    U = env_int("RQMV_BURST_U", 4);
    if (U % S != 0 || (U != 2 && U != 4 && U != 6 && U != 8)) return false;
    const int64_t waves = (rows + U / S - 1) / (U / S);
    grid = (int)((waves + 3) / 4);
    return true;
}

template <int FMT, int M, int U>
static hipError_t launch_burst_u(int xtype, const MvParams& p_in, int S, int grid, hipStream_t stream, hipEvent_t ev0,
                                 hipEvent_t ev1) {
    MvParams p = p_in;
    p.block = 256;
    const size_t lds = matvec_lds_bytes(FMT, xtype, M, p.K);
    auto kernel = xtype == X_F16 ? matvec_burst<FMT, M, U, false> : matvec_burst<FMT, M, U, true>;
    if (lds > 65536) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    if (ev0 || ev1)
        hipExtLaunchKernelGGL(kernel, dim3(grid), dim3(256), (uint32_t)lds, stream, ev0, ev1, 0u, p, S);
    else
        hipLaunchKernelGGL(kernel, dim3(grid), dim3(256), lds, stream, p, S);
    return hipGetLastError();
}

template <int FMT>
static hipError_t launch_burst(int xtype, int M, int U, const MvParams& p, int S, int grid, hipStream_t stream,
                               hipEvent_t ev0, hipEvent_t ev1) {
#define RQ_B(MM, UU) \
    if (M == MM && U == UU) return launch_burst_u<FMT, MM, UU>(xtype, p, S, grid, stream, ev0, ev1);
    RQ_B(1, 2) RQ_B(1, 4) RQ_B(1, 6) RQ_B(1, 8) RQ_B(2, 2) RQ_B(2, 4) RQ_B(2, 6) RQ_B(2, 8)
#undef RQ_B
    return hipErrorInvalidValue;
}

bool try_launch_burst(int fmt, int xtype, int M, const MvParams& p, int cus, hipStream_t stream, hipEvent_t ev0,
                      hipEvent_t ev1, hipError_t* err) {
    int U, S, grid;
    (void)cus;
    if (!burst_plan(fmt, p.rows, p.P.nch, p.P.row_bytes, M, U, S, grid)) return false;
    if (stage_items_host(fmt, p.P.nch, M) > kStageNJ * 256) return false;  // the staging holds four items a thread
    switch (fmt) {
        case Q4_0: *err = launch_burst<Q4_0>(xtype, M, U, p, S, grid, stream, ev0, ev1); break;
        case Q8_0: *err = launch_burst<Q8_0>(xtype, M, U, p, S, grid, stream, ev0, ev1); break;
        case Q4_K: *err = launch_burst<Q4_K>(xtype, M, U, p, S, grid, stream, ev0, ev1); break;
        case Q6_K: *err = launch_burst<Q6_K>(xtype, M, U, p, S, grid, stream, ev0, ev1); break;
        default: return false;
    }
    return true;
}

hipError_t launch_matvec(int fmt, int xtype, int M, const MvParams& p, const LaunchShape& s, hipStream_t stream,
                         hipEvent_t ev0, hipEvent_t ev1) {
    switch (fmt) {
        case Q4_0: return launch_fmt<Q4_0>(xtype, M, p, s, stream, ev0, ev1);
        case Q8_0: return launch_fmt<Q8_0>(xtype, M, p, s, stream, ev0, ev1);
        case Q4_K: return launch_fmt<Q4_K>(xtype, M, p, s, stream, ev0, ev1);
        case Q6_K: return launch_fmt<Q6_K>(xtype, M, p, s, stream, ev0, ev1);
        case F16: return launch_fmt<F16>(xtype, M, p, s, stream, ev0, ev1);
        default: return hipErrorInvalidValue;
    }
}

LaunchShape plan_fused(int fmt, int64_t rows, int64_t cols, int cus, bool glu, bool norm) {
    LaunchShape s;
    // plain products (no prologue, no epilogue) take the plain entry point's
    // two-waves-per-tile form where it applies, with the same shape (so the
    // two entry points stay bit-identical); with the norm prologue or the GLU
    // epilogue too (RQMV_K2_FUSED=0 keeps those in the one-wave form)
    // (the norm prologue's staging takes at most kStageNJNorm items a thread there)
    if ((!glu && !norm) || env_int("RQMV_K2_FUSED", 1))
        if (k2_shape(fmt, rows, chunks_per_row(fmt, cols), 1, X_F32, cus, s) &&
            (!norm || stage_items_host(fmt, chunks_per_row(fmt, cols), 1) <= (int64_t)kStageNJNorm * s.block))
            return s;
    s = plan_matvec_impl(fmt, rows, cols, 1, X_F32, cus, false);
    // a lane group holds a (gate, up) row pair for kEpiGlu; otherwise Q8_0
    // takes one row, as in plan_matvec
    s.R = glu || fmt != Q8_0 ? 2 : 1;
    if (s.block > 512) s.block = 512;
    const int64_t rows_per_wave = (int64_t)(64 / s.G) * s.R;
    const int64_t tiles = (rows + rows_per_wave - 1) / rows_per_wave;
    // One 512-thread workgroup per CU when the product has the tiles for it:
    // every workgroup stages (and, with the prologue, normalises) the whole
    // activation row, so one wide workgroup per CU halves that work against
    // two of 256. Measured on the 32-layer decode step: 535.2 -> 543.9 tok/s
    // (1,024 threads: 506.2). (The standalone 4096 -> 14336 product with fp16
    // x, whose staging is lighter, stays faster at two of 256: 9.8 against
    // 10.3 us.) RQMV_FUSED_WIDE=0 keeps the matvec plan's shape.
    if (env_int("RQMV_FUSED_WIDE", 1) && tiles >= (int64_t)8 * cus) {
        s.block = 512;
        s.grid = cus;
    }
    const int wpb = s.block / 64;
    int64_t grid = (tiles + wpb - 1) / wpb;
    if (grid > s.grid) grid = s.grid;
    s.grid = grid < 1 ? 1 : (int)grid;
    return s;
}

template <int FMT, int R = 2>
static hipError_t launch_fused_fmt(const MvParams& p0, const LaunchShape& s, hipStream_t stream) {
    const size_t lds = matvec_lds_bytes(FMT, X_F32, 1, p0.K);
    MvParams p = p0;
    const int64_t rows_per_wave = (int64_t)(64 / s.G) * R, waves = (int64_t)s.grid * (s.block / 64);
    const int64_t tiles = (p.rows + rows_per_wave - 1) / rows_per_wave;
    // tiles that do not divide over the waves (the decode step's QKV product:
    // 3,072 tiles on 2,048 waves) take the spread numbering: 589.6 -> 594.6
    // tok/s (three alternating runs). RQMV_SPREAD=0 keeps workgroup-major.
    p.spread = env_int("RQMV_SPREAD", 1) != 0 && tiles % waves != 0;
    if (p.norm_w) return launch_kernel(matvec_int<FMT, 1, R, true, true>, p, s, lds, stream, nullptr, nullptr);
    return launch_kernel(matvec_int<FMT, 1, R, true>, p, s, lds, stream, nullptr, nullptr);
}

hipError_t launch_matvec_fused(int fmt, const MvParams& p, const LaunchShape& s, hipStream_t stream) {
    if (s.k2) {  // the two-waves-per-tile form (plan_fused)
        const size_t lds = matvec_lds_bytes(fmt, X_F32, 1, p.K);
        const bool nm = p.norm_w != nullptr;
        auto go = [&](auto plain, auto norm) { return launch_kernel(nm ? norm : plain, p, s, lds, stream, nullptr, nullptr); };
        switch (fmt) {
            case Q4_K: return go(matvec_int_k2<Q4_K, 1, true>, matvec_int_k2<Q4_K, 1, true, 1, true>);
            case Q4_0: return go(matvec_int_k2<Q4_0, 1, true>, matvec_int_k2<Q4_0, 1, true, 1, true>);
            case Q6_K: return go(matvec_int_k2<Q6_K, 1, true>, matvec_int_k2<Q6_K, 1, true, 1, true>);
            case Q8_0: return go(matvec_int_k2<Q8_0, 1, true>, matvec_int_k2<Q8_0, 1, true, 1, true>);
            default: return hipErrorInvalidValue;
        }
    }
    if (s.block > 512) return hipErrorInvalidValue;
    if (s.R == 1 && fmt == Q8_0 && p.epi != kEpiGlu) return launch_fused_fmt<Q8_0, 1>(p, s, stream);
    if (s.R != 2) return hipErrorInvalidValue;
    switch (fmt) {
        case Q4_0: return launch_fused_fmt<Q4_0>(p, s, stream);
        case Q8_0: return launch_fused_fmt<Q8_0>(p, s, stream);
        case Q4_K: return launch_fused_fmt<Q4_K>(p, s, stream);
        case Q6_K: return launch_fused_fmt<Q6_K>(p, s, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_dequant(int fmt, const Planes& P, int64_t rows, int cols, float* out, hipStream_t stream) {
    const int64_t total = rows * P.nch;
    int64_t grid = (total + 255) / 256;
    if (grid > 65536) grid = 65536;
    if (grid < 1) grid = 1;
    switch (fmt) {
        case Q4_0: hipLaunchKernelGGL(dequant_kernel<Q4_0>, dim3(grid), dim3(256), 0, stream, P, rows, cols, out); break;
        case Q8_0: hipLaunchKernelGGL(dequant_kernel<Q8_0>, dim3(grid), dim3(256), 0, stream, P, rows, cols, out); break;
        case Q4_K: hipLaunchKernelGGL(dequant_kernel<Q4_K>, dim3(grid), dim3(256), 0, stream, P, rows, cols, out); break;
        case Q6_K: hipLaunchKernelGGL(dequant_kernel<Q6_K>, dim3(grid), dim3(256), 0, stream, P, rows, cols, out); break;
        case F16: hipLaunchKernelGGL(dequant_kernel<F16>, dim3(grid), dim3(256), 0, stream, P, rows, cols, out); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace rq
