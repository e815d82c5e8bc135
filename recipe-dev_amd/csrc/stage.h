// Activation staging into LDS, shared by the matvec and MoE kernels.
//
// fp16 activations: [m][part][chunk] 16-byte units of eight halves (pairs
// permuted a,c,b,d per run of four when the format's code words hold values
// 4i, 4i+2 / 4i+1, 4i+3 in their two halves), then [m][sum][chunk] fp32 sums of
// consecutive runs of CW/NS activations. fp32 activations: [m][part][chunk]
// 16-byte units of four floats in natural order. Columns at or beyond K read
// as zero. Lanes that take consecutive chunks read consecutive LDS addresses.
#pragma once

#include "chunk.h"

namespace rq {

template <int FMT>
constexpr int xparts16() { return Traits<FMT>::CW / 8; }
template <int FMT>
constexpr int xparts32() { return Traits<FMT>::CW / 4; }
template <int FMT>
constexpr int nsums() { return Traits<FMT>::NS > 0 ? Traits<FMT>::NS : 1; }

template <int FMT>
__device__ __forceinline__ void stage_f16(int nch, int K, const void* xv, int64_t ldx, int M, uint4* xq, float* sums) {
    constexpr int CW = Traits<FMT>::CW, XP = xparts16<FMT>(), NS = Traits<FMT>::NS;
    const uint16_t* x = static_cast<const uint16_t*>(xv);
    const int total = M * XP * nch;
    for (int u = threadIdx.x; u < total; u += blockDim.x) {
        const int c = u % nch, mj = u / nch, j = mj % XP, m = mj / XP;
        const int k0 = c * CW + j * 8;
        const uint16_t* xm = x + (int64_t)m * ldx;
        uint32_t h[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) h[t] = (k0 + t < K) ? xm[k0 + t] : 0u;
        uint4 v;
        if constexpr (Traits<FMT>::PERM4) {
            v = make_uint4(h[0] | (h[2] << 16), h[1] | (h[3] << 16), h[4] | (h[6] << 16), h[5] | (h[7] << 16));
        } else {
            v = make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16));
        }
        xq[u] = v;
    }
    if constexpr (NS > 0) {
        constexpr int GS = CW / NS;
        const int ts = M * NS * nch;
        for (int u = threadIdx.x; u < ts; u += blockDim.x) {
            const int c = u % nch, ms = u / nch, s = ms % NS, m = ms / NS;
            const int k0 = c * CW + s * GS;
            const uint16_t* xm = x + (int64_t)m * ldx;
            float acc = 0.f;
            for (int t = 0; t < GS; ++t)
                if (k0 + t < K) acc += (float)__builtin_bit_cast(_Float16, xm[k0 + t]);
            sums[u] = acc;
        }
    }
}

template <int FMT>
__device__ __forceinline__ void stage_f32(int nch, int K, const void* xv, int64_t ldx, int M, float4* xf) {
    constexpr int CW = Traits<FMT>::CW, XP = xparts32<FMT>();
    const float* x = static_cast<const float*>(xv);
    const int total = M * XP * nch;
    for (int u = threadIdx.x; u < total; u += blockDim.x) {
        const int c = u % nch, mj = u / nch, j = mj % XP, m = mj / XP;
        const int k0 = c * CW + j * 4;
        const float* xm = x + (int64_t)m * ldx;
        float v[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) v[t] = (k0 + t < K) ? xm[k0 + t] : 0.f;
        xf[u] = make_float4(v[0], v[1], v[2], v[3]);
    }
}

// LDS bytes of a staged activation block.
__host__ __device__ inline size_t stage_bytes(int fmt, int xtype_f32, int M, int nch) {
    FormatInfo f = format_info(fmt);
    if (xtype_f32) return (size_t)M * nch * (size_t)(f.chunk_values / 4) * 16;
    return (size_t)M * nch * ((size_t)(f.chunk_values / 8) * 16 + (size_t)(f.sums > 0 ? f.sums : 0) * 4);
}

__device__ __forceinline__ float group_sum(float v, int G) {
    for (int off = G >> 1; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

// Dot of one chunk against staged fp32 activations (exact weights, fma): chunk
// `c` of its weight row, whose activations sit at staged chunk `cx`.
template <int FMT>
__device__ __forceinline__ float chunk_dot_f32(const ChunkData<FMT>& d, int c, const float4* xf, int nch, int cx, int m) {
    constexpr int CW = Traits<FMT>::CW, XP = xparts32<FMT>();
    float w[CW];
    decode_chunk<FMT>(d, c, w);
    float a = 0.f;
#pragma unroll
    for (int j = 0; j < XP; ++j) {
        const float4 xv = xf[(m * XP + j) * nch + cx];
        a = fmaf(w[4 * j], xv.x, a);
        a = fmaf(w[4 * j + 1], xv.y, a);
        a = fmaf(w[4 * j + 2], xv.z, a);
        a = fmaf(w[4 * j + 3], xv.w, a);
    }
    return a;
}

}  // namespace rq
