// Batch-1 and small-M (M <= 8) dequant-dot matrix-vector kernels for gfx950.
//
// Work mapping. A wave's 64 lanes are split into 64/G groups of G lanes; a
// group owns R consecutive rows and its lanes take chunks g, g+G, g+2G, ...
// of those rows, so every load instruction of the wave reads contiguous 16-byte
// parts of the code plane (layout.h). Each lane keeps R x M fp32 partial sums;
// the G lanes of a group are reduced with cross-lane xor shuffles (no atomics,
// no scratch) and the first lane writes the rows. Waves stride over row tiles,
// so a fixed, occupancy-sized grid covers any row count.
//
// Activations are staged once per workgroup into LDS, in a part-major layout
// ([m][part][chunk] 16-byte units) that makes the lanes' LDS reads
// conflict-free, together with the per-chunk activation sums that the fp16
// form needs (chunk.h).
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

template <int FMT, int M, int R>
__global__ void __launch_bounds__(256) matvec_f16(MvParams p) {
    constexpr int XP = xparts16<FMT>(), NS = nsums<FMT>();
    extern __shared__ uint4 smem[];
    const int nch = p.P.nch;
    uint4* xq = smem;
    float* sums = reinterpret_cast<float*>(smem + M * XP * nch);
    stage_f16<FMT>(nch, p.K, p.x, p.ldx, M, xq, sums);
    __syncthreads();

    const int G = p.G;
    const int lane = threadIdx.x & 63, g = lane & (G - 1), sub = lane / G;
    const int wpb = blockDim.x >> 6, wave = threadIdx.x >> 6;
    const int64_t rows_per_wave = (int64_t)(64 / G) * R;
    const int64_t tiles = (p.rows + rows_per_wave - 1) / rows_per_wave;
    for (int64_t tile = (int64_t)blockIdx.x * wpb + wave; tile < tiles; tile += (int64_t)gridDim.x * wpb) {
        const int64_t row0 = tile * rows_per_wave + (int64_t)sub * R;
        float acc[R][M];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int m = 0; m < M; ++m) acc[r][m] = 0.f;
        for (int c = g; c < nch; c += G) {
            uint4 xv[M][XP];
            float sv[M][NS];
#pragma unroll
            for (int m = 0; m < M; ++m) {
#pragma unroll
                for (int j = 0; j < XP; ++j) xv[m][j] = xq[(m * XP + j) * nch + c];
#pragma unroll
                for (int s = 0; s < NS; ++s) sv[m][s] = (Traits<FMT>::NS > 0) ? sums[(m * NS + s) * nch + c] : 0.f;
            }
            ChunkData<FMT> d[R];
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (row0 + r < p.rows) load_chunk<FMT>(p.P, row0 + r, c, d[r]);
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (row0 + r < p.rows) dot_f16<FMT, M>(d[r], c, xv, sv, acc[r]);
        }
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int m = 0; m < M; ++m) acc[r][m] = group_sum(acc[r][m], G);
        if (g == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (row0 + r < p.rows)
#pragma unroll
                    for (int m = 0; m < M; ++m) p.y[(int64_t)m * p.ldy + row0 + r] = acc[r][m];
        }
    }
}

template <int FMT, int M, int R>
__global__ void __launch_bounds__(256) matvec_f32(MvParams p) {
    extern __shared__ float4 smemf[];
    const int nch = p.P.nch;
    stage_f32<FMT>(nch, p.K, p.x, p.ldx, M, smemf);
    __syncthreads();

    const int G = p.G;
    const int lane = threadIdx.x & 63, g = lane & (G - 1), sub = lane / G;
    const int wpb = blockDim.x >> 6, wave = threadIdx.x >> 6;
    const int64_t rows_per_wave = (int64_t)(64 / G) * R;
    const int64_t tiles = (p.rows + rows_per_wave - 1) / rows_per_wave;
    for (int64_t tile = (int64_t)blockIdx.x * wpb + wave; tile < tiles; tile += (int64_t)gridDim.x * wpb) {
        const int64_t row0 = tile * rows_per_wave + (int64_t)sub * R;
        float acc[R][M];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int m = 0; m < M; ++m) acc[r][m] = 0.f;
        for (int c = g; c < nch; c += G) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                if (row0 + r >= p.rows) continue;
                ChunkData<FMT> d;
                load_chunk<FMT>(p.P, row0 + r, c, d);
#pragma unroll
                for (int m = 0; m < M; ++m) acc[r][m] += chunk_dot_f32<FMT>(d, c, smemf, nch, c, m);
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int m = 0; m < M; ++m) acc[r][m] = group_sum(acc[r][m], G);
        if (g == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (row0 + r < p.rows)
#pragma unroll
                    for (int m = 0; m < M; ++m) p.y[(int64_t)m * p.ldy + row0 + r] = acc[r][m];
        }
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
    return stage_bytes(fmt, xtype == X_F32, M, (int)chunks_per_row(fmt, cols));
}

static int env_int(const char* name, int fallback) {
    const char* v = getenv(name);
    return v && *v ? atoi(v) : fallback;
}

LaunchShape plan_matvec(int fmt, int64_t rows, int64_t cols, int M, int xtype, int cus) {
    LaunchShape s;
    const int64_t nch = chunks_per_row(fmt, cols);
    int G = 64;
    while (G > 8 && G > nch) G >>= 1;
    s.G = G;
    s.R = M == 1 ? 4 : (M == 2 ? 2 : 1);
    if (xtype == X_F32) s.R = M == 1 ? 2 : 1;
    s.block = 256;
    s.G = env_int("RQMV_G", s.G);
    s.R = env_int("RQMV_R", s.R);
    s.block = env_int("RQMV_BLOCK", s.block);
    const int64_t rows_per_wave = (int64_t)(64 / s.G) * s.R;
    const int64_t tiles = (rows + rows_per_wave - 1) / rows_per_wave;
    const int wpb = s.block / 64;
    int64_t grid = (tiles + wpb - 1) / wpb;
    const int64_t cap = (int64_t)cus * env_int("RQMV_BLOCKS_PER_CU", 8);
    if (grid > cap) grid = cap;
    s.grid = env_int("RQMV_GRID", (int)grid);
    if (s.grid < 1) s.grid = 1;
    return s;
}

template <int FMT, int M, int R>
static hipError_t launch_one(int xtype, const MvParams& p, const LaunchShape& s, hipStream_t stream, hipEvent_t ev0,
                             hipEvent_t ev1) {
    const size_t lds = matvec_lds_bytes(FMT, xtype, M, p.K);
    const void* fn = xtype == X_F16 ? reinterpret_cast<const void*>(&matvec_f16<FMT, M, R>)
                                    : reinterpret_cast<const void*>(&matvec_f32<FMT, M, R>);
    if (lds > 65536) {
        hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    if (ev0 || ev1) {
        // Events recorded by the dispatch itself: its start and completion times.
        if (xtype == X_F16)
            hipExtLaunchKernelGGL((matvec_f16<FMT, M, R>), dim3(s.grid), dim3(s.block), (uint32_t)lds, stream, ev0, ev1,
                                  0u, p);
        else
            hipExtLaunchKernelGGL((matvec_f32<FMT, M, R>), dim3(s.grid), dim3(s.block), (uint32_t)lds, stream, ev0, ev1,
                                  0u, p);
    } else if (xtype == X_F16) {
        hipLaunchKernelGGL((matvec_f16<FMT, M, R>), dim3(s.grid), dim3(s.block), lds, stream, p);
    } else {
        hipLaunchKernelGGL((matvec_f32<FMT, M, R>), dim3(s.grid), dim3(s.block), lds, stream, p);
    }
    return hipGetLastError();
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
        case 64 + 1: return launch_one<FMT, 4, 1>(xtype, p, s, stream, ev0, ev1);
        case 128 + 1: return launch_one<FMT, 8, 1>(xtype, p, s, stream, ev0, ev1);
        default: return hipErrorInvalidValue;
    }
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
