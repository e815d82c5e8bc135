// Internal launch interface between the C-ABI layer and the HIP kernels.
#pragma once

#include <hip/hip_runtime.h>

#include "chunk.h"

namespace rq {

enum XType : int { X_F32 = 0, X_F16 = 1 };

// A matrix-vector product over a repacked weight: y[m*ldy + n] =
// sum_k W[n][k] x[m*ldx + k] for n < rows, m < M.
struct MvParams {
    Planes P;
    int64_t rows;
    int K;
    const void* x;
    int64_t ldx;
    float* y;
    int64_t ldy;
    int G;  // lanes that share one row (power of two, 8..64)
    int block = 256;  // threads per workgroup (the launch's block size)
    // The row-tile walk of the vector kernels, set by the launcher from the
    // launch shape (so that no wave divides before its first load): log2 G,
    // rows per wave tile ((64 / G) * R), row tiles, and steps per tile
    // (ceil(chunks / G)).
    int g_shift = 6;
    int rows_per_wave = 1;
    int tiles = 0;
    int steps = 1;
    // 1: first tiles numbered SIMD-group-major across the workgroups (matvec.hip
    // make_walk), for launches whose tiles do not divide evenly over the waves
    int spread = 0;
    // F16 weights only: rows at or past `split` come from P2 (row - split), so
    // that two weights of one width run as one launch (an MoE router and its
    // shared-expert gate). split >= rows: P alone.
    Planes P2;
    int64_t split;
    // Decode-step fusions (quantized weights, one fp32 activation row):
    // prologue (norm_w set): x is read as u = x + delta (delta optional), u is
    // written to x_out (when set, by workgroup 0), and the product takes
    // rmsnorm(u) * norm_w = u * norm_w / sqrt(sum u^2 / K + eps), the common
    // factor applied to the finished products; epilogue (epi): kEpiPlain
    // writes y, kEpiGlu takes rows as (gate, up) pairs and writes
    // y[i] = silu(row 2i) * row 2i+1.
    int epi = 0;
    const float* norm_w = nullptr;
    const float* delta = nullptr;
    float* x_out = nullptr;
    float eps = 0.f;
};

enum Epilogue : int { kEpiPlain = 0, kEpiGlu = 1 };

struct LaunchShape {
    int G = 64;       // lanes per row group
    int R = 1;        // rows per lane group per tile
    int block = 256;  // threads per workgroup
    int grid = 0;     // workgroups (0 = derive)
    bool k2 = false;  // two waves per row tile (matvec_int_k2)
};

// Chooses G, R, block and grid for a product; honours RQMV_G / RQMV_R /
// RQMV_BLOCK / RQMV_GRID overrides for tuning sweeps.
LaunchShape plan_matvec(int fmt, int64_t rows, int64_t cols, int M, int xtype, int cus);
// Whether a product of M activation rows takes two waves per row tile (matvec_int_k2).
bool k2_takes(int fmt, int64_t rows, int64_t cols, int M, int xtype, int cus);

// ev0 / ev1 (may be null): events the dispatch records at its start and end.
hipError_t launch_matvec(int fmt, int xtype, int M, const MvParams& p, const LaunchShape& s, hipStream_t stream,
                         hipEvent_t ev0 = nullptr, hipEvent_t ev1 = nullptr);

// The burst form of the M <= 2 integer product (long rows, every weight load
// issued at launch), when it applies: returns false (nothing launched) when
// the shape does not suit it, else launches and puts the result in *err.
bool try_launch_burst(int fmt, int xtype, int M, const MvParams& p, int cus, hipStream_t stream, hipEvent_t ev0,
                      hipEvent_t ev1, hipError_t* err);

// Exact fp32 decode of every weight, rows x cols in GGUF order.
hipError_t launch_dequant(int fmt, const Planes& P, int64_t rows, int cols, float* out, hipStream_t stream);

size_t matvec_lds_bytes(int fmt, int xtype, int M, int cols);

// The decode-step fused product (M = 1, fp32 activations, quantized weight):
// the launch shape it uses and the launch itself.
LaunchShape plan_fused(int fmt, int64_t rows, int64_t cols, int cus, bool glu, bool norm);
hipError_t launch_matvec_fused(int fmt, const MvParams& p, const LaunchShape& s, hipStream_t stream);

// Matrix-core product for 1 <= M <= 32 activation rows (quantized formats).
hipError_t launch_matvec_mfma(int fmt, int xtype, int M, const MvParams& p, int cus, hipStream_t stream,
                              hipEvent_t ev0 = nullptr, hipEvent_t ev1 = nullptr);
size_t mfma_lds_bytes(int fmt, int xtype, int M, int64_t rows, int cus);

// recipe's int(8) sum (int8.hip): Q8 activation records of `step` (32 or 256)
// inputs, v_dot4_i32_i8 block dots, recipe's fp32 order. y[m*ldy + n] for
// n < rows, m < M; tail: the last position folds 256-step Q4_K blocks whole.
size_t int8_lds_bytes(int64_t cols);
hipError_t launch_matvec_int8(int fmt, const Planes& P, int64_t rows, int K, const float* x, int M, int64_t ldx,
                              float* y, int64_t ldy, int step, int tail, hipStream_t stream);
hipError_t launch_q8_records(const float* x, int K, int step, float* d, int8_t* codes, hipStream_t stream);

}  // namespace rq
