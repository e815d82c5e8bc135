// Small-M (2 <= M <= 32) quantized products on the matrix cores of gfx950:
// the kernels (included by mfma.hip, fp16 activations, and mfma_f32.hip, fp32
// activations, which are built with different code-generation options).
//
// y[m][n] = sum_k W[n][k] x[m][k] is a real contraction once M > 1: each
// weight is used M times. Here the weights are decoded to their exact
// integer codes in fp16 (q, q - 8 or q - 32 are small integers, exact in
// fp16) and multiplied with the fp16 activations on v_mfma_f32_16x16x32_f16
// (v_mfma_f32_16x16x16_f16 for Q6_K, whose scales cover 16 weights). Every
// product is exact and the matrix core accumulates one scale block in fp32;
// the block's scale is applied to that block's 16x16 result in fp32 (and for
// Q4_K the minimum through a second product of x with a block of ones), so
// the arithmetic matches the batch-1 kernels' per-block epilogue. fp32
// activations are first scaled per (scale block, activation row) by the power
// of two that brings the block's largest magnitude into [2^14, 2^15), then
// split into an fp16 high and low part (x = hi + lo to 2^-22 of the value, or
// 2^-39 of the block's largest) and multiplied as two tiles; the inverse power
// multiplies the block's scaled result, so no value overflows fp16 or loses
// its low bits to fp16's subnormal range.
//
// Work mapping. A workgroup of W waves (four, or fewer for short matrices)
// owns 16 W rows (16 per wave, the matrix core's N) and walks K in sub-steps of four chunks (256 weights, 128
// for Q8_0):
//   * the sub-step's activations, all M rows, are staged once per workgroup
//     into LDS in the matrix core's A-operand order (double-buffered);
//   * each wave loads its 16 rows x 256 weights with the same 16-byte,
//     row-contiguous loads as the batch-1 kernels (lane = row, chunk), four
//     sub-steps ahead of their use, decodes them and writes them to its own LDS
//     tile in the B-operand order (the transpose from chunk-per-lane to
//     k-slice-per-lane), with one fp32 scale pair per (block, row);
//   * each 32-weight block (16 for Q6_K) is one MFMA per 16 activation rows
//     into a zeroed accumulator, added into the running sums with its scale.
// Reference counterpart: packed_lanes4_body (amd-nv-cpu.ll:2674-3126) and the
// general contraction body (amd-nv-cpu.ll:3509-3649), which take M > 1 in fp32
// fma on the vector units.
#pragma once

#include <hip/hip_ext.h>
#include <stdlib.h>

#include <type_traits>

#include "halfcode.h"
#include "kernels.h"

namespace rq {


// A sub-step is four chunks of every row (SUBK weights of K: 256, or 128 for
// Q8_0), one chunk per loader lane; NB matrix-core blocks per sub-step, KB
// weights per block (the MFMA's K).
template <int FMT> struct MfmaTraits;
template <> struct MfmaTraits<Q4_0> { static constexpr int SUBK = 256, NB = 8, KB = 32; };
template <> struct MfmaTraits<Q4_K> { static constexpr int SUBK = 256, NB = 8, KB = 32; };
template <> struct MfmaTraits<Q8_0> { static constexpr int SUBK = 128, NB = 4, KB = 32; };
template <> struct MfmaTraits<Q6_K> { static constexpr int SUBK = 256, NB = 16, KB = 16; };

constexpr int kWeightDepth = 4; // sub-steps of weights in flight per wave
constexpr int kUnitPad = 17;    // B-tile units per (block, k-slice): 16 rows + 1 against bank conflicts

template <int FMT, int NT, bool XF32, int W>
struct MfmaLds {
    using T = MfmaTraits<FMT>;
    static constexpr int NTA = NT * (XF32 ? 2 : 1);           // A tiles per block (hi/lo for fp32 x)
    static constexpr int UB = T::KB == 32 ? 16 : 8;           // bytes per operand unit (8 or 4 halves)
    static constexpr int XSC = XF32 ? T::NB * NT * 16 * 4 : 0;  // fp32 x: a power of two per (block, row)
    static constexpr int XBUF = T::NB * NTA * 64 * UB + XSC;  // one staged activation sub-step
    static constexpr int BTILE = T::NB * 4 * kUnitPad * UB + 128;   // one wave's decoded weights (+ skew)
    static constexpr int SCALES = T::NB * 16 * 8 + 128;             // one wave's (scale, min) pairs (+ skew)
    static constexpr int WAVE = BTILE + SCALES;
    static constexpr int TOTAL = 2 * XBUF + W * WAVE;
};

// fp32 activations: the exponent k that brings a block's largest magnitude
// `amax` into [2^14, 2^15) (fp16 holds up to 65504), 0 for a zero or
// non-finite block, within [-126, 126] so that 2^-k is a normal fp32.
__device__ __forceinline__ int block_shift(float amax) {
    if (!(amax > 0.f) || !(amax <= 3.402823466e38f)) return 0;
    const int k = 15 - __builtin_amdgcn_frexp_expf(amax);
    return k < -126 ? -126 : (k > 126 ? 126 : k);
}

// x * 2^k split into an fp16 high part and the fp16 rounding of the rest.
__device__ __forceinline__ void split_scaled(float x, int k, _Float16& hi, _Float16& lo) {
    const float v = __builtin_amdgcn_ldexpf(x, k);
    hi = (_Float16)v;
    lo = (_Float16)(v - (float)hi);
}

// Byte offset of B-tile unit (block b, k-slice q, row n). The blocks of one
// loader chunk are shifted by 32 bytes per chunk, so that the four loader
// lanes of a row (same n, different chunk) write to different LDS banks.
template <int FMT>
__device__ __forceinline__ int bt_unit(int b, int q, int n) {
    using T = MfmaTraits<FMT>;
    constexpr int UB = T::KB == 32 ? 16 : 8, PER_CHUNK = T::NB / 4;
    return ((b * 4 + q) * kUnitPad + n) * UB + (b / PER_CHUNK) * 32;
}
template <int FMT>
__device__ __forceinline__ int scl_index(int b, int n) {
    constexpr int PER_CHUNK = MfmaTraits<FMT>::NB / 4;
    return b * 16 + n + (b / PER_CHUNK) * 4;  // float2 units: 32-byte shift per chunk
}

// Decodes one loader lane's chunk (row ln, chunk lj of the sub-step) into a
// wave's B tile and scale table.
template <int FMT>
__device__ __forceinline__ void decode_to_tile(const ChunkData<FMT>& d0, int ln, int lj, uint8_t* bt, float2* scl) {
    if constexpr (FMT == Q4_0 || FMT == Q4_K) {
        const uint32_t neg = FMT == Q4_0 ? 0xD480E408u : 0xD400E400u;  // (-1032, -72) or (-1024, -64)
#pragma unroll
        for (int part = 0; part < 2; ++part) {
            const int b = 2 * lj + part;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                uint32_t o[4];
                nibbles_to_h(word(d0.q[part], q) ^ 0x88888888u, neg, o);
                *reinterpret_cast<uint4*>(bt + bt_unit<FMT>(b, q, ln)) = make_uint4(o[0], o[1], o[2], o[3]);
            }
        }
        if constexpr (FMT == Q4_K) {
            uint32_t sc0, m0, sc1, m1;
            q4k_scales(d0.meta, lj, sc0, m0, sc1, m1);
            const float dd = half_lo(d0.meta.x), dmin = half_hi(d0.meta.x);
            scl[scl_index<FMT>(2 * lj, ln)] = make_float2(dd * (float)sc0, dmin * (float)m0);
            scl[scl_index<FMT>(2 * lj + 1, ln)] = make_float2(dd * (float)sc1, dmin * (float)m1);
        } else {
            scl[scl_index<FMT>(2 * lj, ln)] = make_float2(half_lo(d0.meta.x), 0.f);
            scl[scl_index<FMT>(2 * lj + 1, ln)] = make_float2(half_hi(d0.meta.x), 0.f);
        }
    } else if constexpr (FMT == Q8_0) {
        const int b = lj;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            uint32_t o[4];
            bytes_to_h(word(d0.q[q >> 1], 2 * (q & 1)), o[0], o[1]);
            bytes_to_h(word(d0.q[q >> 1], 2 * (q & 1) + 1), o[2], o[3]);
            *reinterpret_cast<uint4*>(bt + bt_unit<FMT>(b, q, ln)) = make_uint4(o[0], o[1], o[2], o[3]);
        }
        scl[scl_index<FMT>(b, ln)] = make_float2(half_lo(d0.meta.x), 0.f);
    } else {  // Q6_K: four 16-weight scale groups per chunk
        const float dd = half_lo(d0.meta.y);
#pragma unroll
        for (int gg = 0; gg < 4; ++gg) {
            const int g = 4 * lj + gg;
            const uint32_t L0 = word(d0.q[gg >> 1], (gg & 1) * 2) ^ 0x88888888u;
            const uint32_t L1 = word(d0.q[gg >> 1], (gg & 1) * 2 + 1) ^ 0x88888888u;
            const uint32_t H = word(d0.q[2], gg);
            uint32_t o[4], o2[4];
            q6_to_h(L0, H & 0x33333333u, o);
            q6_to_h(L1, (H >> 2) & 0x33333333u, o2);
            *reinterpret_cast<uint2*>(bt + bt_unit<FMT>(g, 0, ln)) = make_uint2(o[0], o[1]);
            *reinterpret_cast<uint2*>(bt + bt_unit<FMT>(g, 1, ln)) = make_uint2(o[2], o[3]);
            *reinterpret_cast<uint2*>(bt + bt_unit<FMT>(g, 2, ln)) = make_uint2(o2[0], o2[1]);
            *reinterpret_cast<uint2*>(bt + bt_unit<FMT>(g, 3, ln)) = make_uint2(o2[2], o2[3]);
            scl[scl_index<FMT>(g, ln)] = make_float2(dd * (float)(int8_t)((d0.meta.x >> (8 * gg)) & 0xffu), 0.f);
        }
    }
}

template <int FMT, int NT, bool XF32, int W>
__global__ void __launch_bounds__(64 * W) matvec_mfma(MvParams p, int M, uint32_t x_bytes) {
    using TR = MfmaTraits<FMT>;
    using L = MfmaLds<FMT, NT, XF32, W>;
    constexpr int SUBK = TR::SUBK, NB = TR::NB, NTA = L::NTA;
    constexpr int XI = 16 * NT * (SUBK / 8) / (64 * W);  // activation items per thread
    constexpr int XW = XF32 ? 2 : 1;                                // 16-byte loads per item
    extern __shared__ uint4 smem[];
    uint8_t* lds = reinterpret_cast<uint8_t*>(smem);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint8_t* const xbuf[2] = {lds, lds + L::XBUF};
    uint8_t* const bt = lds + 2 * L::XBUF + wave * L::WAVE;
    float2* const scl = reinterpret_cast<float2*>(bt + L::BTILE);

    const int64_t row0 = ((int64_t)blockIdx.x * W + wave) * 16;
    const int nch = p.P.nch;
    const int steps = (nch + 3) / 4;
    const __amdgpu_buffer_rsrc_t rs = planes_rsrc(p.P);
    const __amdgpu_buffer_rsrc_t xrs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p.x), (short)0, (int)x_bytes, 0x00020000);
    const int ln = lane >> 2, lj = lane & 3;          // loader: row, chunk of the sub-step
    const int mn = lane & 15, mq = lane >> 4;         // matrix core: B column (row n), k-slice
    const int64_t lrow = row0 + ln;
    const bool lrow_ok = lrow < p.rows;

    auto load_w = [&](int t, ChunkData<FMT>& d) {
        const int c = t * 4 + lj;
        load_chunk_rs<FMT>(rs, p.P, (uint32_t)lrow, c, lrow_ok && c < nch, d);
    };
    // Activation item of a sub-step: eight values at k8 * 8 of row mm = 16 tm
    // + m, with m fastest so that consecutive lanes write consecutive LDS units.
    constexpr int K8 = SUBK / 8;
    auto load_x = [&](int t, uint4 (&v)[XI][XW]) {
#pragma unroll
        for (int i = 0; i < XI; ++i) {
            const int item = (int)threadIdx.x + 64 * W * i;
            const int mm = ((item >> 4) / K8) * 16 + (item & 15), k = t * SUBK + 8 * ((item >> 4) % K8);
            const bool ok = mm < M && k < p.K;
            const uint32_t off = (uint32_t)(((int64_t)mm * p.ldx + k) * (XF32 ? 4 : 2));
#pragma unroll
            for (int h = 0; h < XW; ++h) {
                const u32x4_t r = __builtin_amdgcn_raw_buffer_load_b128(xrs, ok ? off + 16u * h : kOobOffset, 0, 0);
                v[i][h] = make_uint4(r.x, r.y, r.z, r.w);
            }
        }
    };
    auto store_x = [&](const uint4 (&v)[XI][XW], uint8_t* xb) {
#pragma unroll
        for (int i = 0; i < XI; ++i) {
            const int item = (int)threadIdx.x + 64 * W * i;
            const int m = item & 15, k8 = (item >> 4) % K8, tm = (item >> 4) / K8;
            uint4 parts[2];  // [0] = fp16 values (or the high parts), [1] = low parts
            if constexpr (XF32) {
                uint32_t hi[4], lo[4];
                const float f[8] = {__builtin_bit_cast(float, v[i][0].x), __builtin_bit_cast(float, v[i][0].y),
                                    __builtin_bit_cast(float, v[i][0].z), __builtin_bit_cast(float, v[i][0].w),
                                    __builtin_bit_cast(float, v[i][1].x), __builtin_bit_cast(float, v[i][1].y),
                                    __builtin_bit_cast(float, v[i][1].z), __builtin_bit_cast(float, v[i][1].w)};
                // the block's largest magnitude: its items sit in lanes 16 apart
                // (k8 = 4b + lane / 16 for 32-weight blocks, 2g + lane / 16 for 16)
                float am = 0.f;
#pragma unroll
                for (int e = 0; e < 8; ++e) am = fmaxf(am, fabsf(f[e]));
                am = fmaxf(am, __shfl_xor(am, 16));
                if constexpr (TR::KB == 32) am = fmaxf(am, __shfl_xor(am, 32));
                const int ks = block_shift(am);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    _Float16 h0, h1, l0, l1;
                    split_scaled(f[2 * e], ks, h0, l0);
                    split_scaled(f[2 * e + 1], ks, h1, l1);
                    hi[e] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
                    lo[e] = (uint32_t)__builtin_bit_cast(uint16_t, l0) | ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
                }
                parts[0] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
                parts[1] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
                const int blk = TR::KB == 32 ? k8 >> 2 : k8 >> 1;
                if ((k8 & (TR::KB == 32 ? 3 : 1)) == 0)
                    reinterpret_cast<float*>(xb + L::XBUF - L::XSC)[(blk * NT + tm) * 16 + m] =
                        __builtin_amdgcn_ldexpf(1.0f, -ks);
            } else {
                parts[0] = v[i][0];
            }
#pragma unroll
            for (int h = 0; h < XW; ++h) {
                const int ta = tm * XW + h;
                if constexpr (TR::KB == 32) {
                    const int b = k8 >> 2, q = k8 & 3;
                    *reinterpret_cast<uint4*>(xb + (((b * NTA + ta) * 64) + q * 16 + m) * 16) = parts[h];
                } else {
                    const int g = k8 >> 1, q = 2 * (k8 & 1);
                    *reinterpret_cast<uint2*>(xb + (((g * NTA + ta) * 64) + q * 16 + m) * 8) = make_uint2(parts[h].x, parts[h].y);
                    *reinterpret_cast<uint2*>(xb + (((g * NTA + ta) * 64) + (q + 1) * 16 + m) * 8) = make_uint2(parts[h].z, parts[h].w);
                }
            }
        }
    };
    auto store_b = [&](const ChunkData<FMT>& d0) { decode_to_tile<FMT>(d0, ln, lj, bt, scl); };

    f4_t acc[NT];
#pragma unroll
    for (int ta = 0; ta < NT; ++ta) acc[ta] = f4_t{0.f, 0.f, 0.f, 0.f};

    // The sub-step's products: one matrix-core block at a time, scaled into acc.
    auto multiply = [&](const uint8_t* xb) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const float2 s = scl[scl_index<FMT>(b, mn)];
            if constexpr (TR::KB == 32) {
                const h8_t B = *reinterpret_cast<const h8_t*>(bt + bt_unit<FMT>(b, mq, mn));
#pragma unroll
                for (int ta = 0; ta < NT; ++ta) {
                    const f4_t z = {0.f, 0.f, 0.f, 0.f};
                    f4_t D, D2;
                    if constexpr (XF32) {
                        const h8_t Ah = *reinterpret_cast<const h8_t*>(xb + ((b * NTA + 2 * ta) * 64 + lane) * 16);
                        const h8_t Al = *reinterpret_cast<const h8_t*>(xb + ((b * NTA + 2 * ta + 1) * 64 + lane) * 16);
                        D = __builtin_amdgcn_mfma_f32_16x16x32_f16(Al, B, __builtin_amdgcn_mfma_f32_16x16x32_f16(Ah, B, z, 0, 0, 0), 0, 0, 0);
                        if constexpr (FMT == Q4_K) {
                            const h8_t one = {1, 1, 1, 1, 1, 1, 1, 1};
                            D2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(Al, one, __builtin_amdgcn_mfma_f32_16x16x32_f16(Ah, one, z, 0, 0, 0), 0, 0, 0);
                        }
                    } else {
                        const h8_t A = *reinterpret_cast<const h8_t*>(xb + ((b * NTA + ta) * 64 + lane) * 16);
                        D = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B, z, 0, 0, 0);
                        if constexpr (FMT == Q4_K) {
                            const h8_t one = {1, 1, 1, 1, 1, 1, 1, 1};
                            D2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, one, z, 0, 0, 0);
                        }
                    }
                    if constexpr (XF32) {
                        // the block's scaled result, times the inverse power of its activation rows
                        const f4_t fx = *reinterpret_cast<const f4_t*>(xb + L::XBUF - L::XSC + ((b * NT + ta) * 16 + 4 * mq) * 4);
#pragma unroll
                        for (int j = 0; j < 4; ++j) {  // (the power of two folds exactly into the scales)
                            float a = fmaf(s.x * fx[j], D[j], acc[ta][j]);
                            if constexpr (FMT == Q4_K) a = fmaf(-s.y * fx[j], D2[j], a);
                            acc[ta][j] = a;
                        }
                    } else {
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            float a = fmaf(s.x, D[j], acc[ta][j]);
                            if constexpr (FMT == Q4_K) a = fmaf(-s.y, D2[j], a);
                            acc[ta][j] = a;
                        }
                    }
                }
            } else {
                const h4_t B = *reinterpret_cast<const h4_t*>(bt + bt_unit<FMT>(b, mq, mn));
#pragma unroll
                for (int ta = 0; ta < NT; ++ta) {
                    const f4_t z = {0.f, 0.f, 0.f, 0.f};
                    f4_t D;
                    if constexpr (XF32) {
                        const h4_t Ah = *reinterpret_cast<const h4_t*>(xb + ((b * NTA + 2 * ta) * 64 + lane) * 8);
                        const h4_t Al = *reinterpret_cast<const h4_t*>(xb + ((b * NTA + 2 * ta + 1) * 64 + lane) * 8);
                        D = __builtin_amdgcn_mfma_f32_16x16x16f16(Al, B, __builtin_amdgcn_mfma_f32_16x16x16f16(Ah, B, z, 0, 0, 0), 0, 0, 0);
                    } else {
                        const h4_t A = *reinterpret_cast<const h4_t*>(xb + ((b * NTA + ta) * 64 + lane) * 8);
                        D = __builtin_amdgcn_mfma_f32_16x16x16f16(A, B, z, 0, 0, 0);
                    }
                    if constexpr (XF32) {
                        const f4_t fx = *reinterpret_cast<const f4_t*>(xb + L::XBUF - L::XSC + ((b * NT + ta) * 16 + 4 * mq) * 4);
#pragma unroll
                        for (int j = 0; j < 4; ++j) acc[ta][j] = fmaf(s.x * fx[j], D[j], acc[ta][j]);
                    } else {
#pragma unroll
                        for (int j = 0; j < 4; ++j) acc[ta][j] = fmaf(s.x, D[j], acc[ta][j]);
                    }
                }
            }
        }
    };

    // Weights run kWeightDepth sub-steps ahead in rotating register sets and
    // activations two sub-steps ahead (a register set, then an LDS buffer), so
    // that enough bytes are in flight to cover HBM latency. A set is refilled
    // only after it has been decoded, never copied while its loads are pending.
    ChunkData<FMT> w[kWeightDepth];
    uint4 xr[2][XI][XW];
    load_x(0, xr[0]);
    load_x(1, xr[1]);
#pragma unroll
    for (int i = 0; i < kWeightDepth; ++i) load_w(i, w[i]);
    store_x(xr[0], xbuf[0]);
    __syncthreads();
    // whole rounds of kWeightDepth sub-steps: the ones past K load nothing
    // (out-of-range buffer loads) and add zero
    const int rounds = (steps + kWeightDepth - 1) / kWeightDepth;
    for (int r = 0; r < rounds; ++r) {
#pragma unroll
        for (int u = 0; u < kWeightDepth; ++u) {
            const int t = r * kWeightDepth + u;
            load_x(t + 2, xr[u & 1]);
            store_b(w[u]);
            asm volatile("" ::: "memory");  // the tile is read back under other types
            multiply(xbuf[u & 1]);
            load_w(t + kWeightDepth, w[u]);
            store_x(xr[(u + 1) & 1], xbuf[(u + 1) & 1]);
            __syncthreads();
        }
    }

    const int64_t row = row0 + mn;
    if (row < p.rows) {
#pragma unroll
        for (int ta = 0; ta < NT; ++ta)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int m = 16 * ta + 4 * mq + j;
                if (m < M) p.y[(int64_t)m * p.ldy + row] = acc[ta][j];
            }
    }
}

// Split-K form for M <= 16 rows of fp16 activations. A workgroup of
// kSplitK waves owns one 16-row stripe and its waves take interleaved
// sub-steps of K, so a matrix of N rows runs N/16 x kSplitK independent waves
// with no barrier inside the loop. Each lane loads its own matrix-core A
// fragments (eight or four activation values per block) straight from the
// cache hierarchy; the weights go through the wave's LDS tile as above. The
// waves' 16x16 partial sums are added in wave order at the end.
constexpr int kSplitK = 4;

template <int FMT>
struct SkLds {
    using T = MfmaTraits<FMT>;
    static constexpr int UB = T::KB == 32 ? 16 : 8;
    static constexpr int BTILE = T::NB * 4 * kUnitPad * UB + 128;
    static constexpr int SCALES = T::NB * 16 * 8 + 128;
    static constexpr int WAVE = BTILE + SCALES;
    static constexpr int RED = kSplitK * 64 * 16;  // partial sums, one f4 per lane and wave
    static constexpr int TOTAL = kSplitK * WAVE + RED;
};

template <int FMT>
__global__ void __launch_bounds__(64 * kSplitK) matvec_mfma_sk(MvParams p, int M, uint32_t x_bytes) {
    using TR = MfmaTraits<FMT>;
    using L = SkLds<FMT>;
    constexpr int SUBK = TR::SUBK, NB = TR::NB, KB = TR::KB;
    constexpr int DW = kWeightDepth;
    extern __shared__ uint4 smem[];
    uint8_t* lds = reinterpret_cast<uint8_t*>(smem);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint8_t* const bt = lds + wave * L::WAVE;
    float2* const scl = reinterpret_cast<float2*>(bt + L::BTILE);
    f4_t* const red = reinterpret_cast<f4_t*>(lds + kSplitK * L::WAVE);

    const int64_t row0 = (int64_t)blockIdx.x * 16;
    const int nch = p.P.nch;
    const int steps = (nch + 3) / 4;
    const __amdgpu_buffer_rsrc_t rs = planes_rsrc(p.P);
    const __amdgpu_buffer_rsrc_t xrs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p.x), (short)0, (int)x_bytes, 0x00020000);
    const int ln = lane >> 2, lj = lane & 3;   // loader: row, chunk of the sub-step
    const int mn = lane & 15, mq = lane >> 4;  // matrix core: row n / activation row m, k-slice
    const int64_t lrow = row0 + ln;
    const bool lrow_ok = lrow < p.rows;
    const uint32_t xkeep = mn < M ? 0xFFFFFFFFu : 0u;

    auto load_w = [&](int t, ChunkData<FMT>& d) {
        const int c = t * 4 + lj;
        load_chunk_rs<FMT>(rs, p.P, (uint32_t)lrow, c, lrow_ok && c < nch, d);
    };
    // A fragment of block b of sub-step t: activation row mn, values KB/4
    // starting at k = t * SUBK + KB * b + (KB / 4) * mq.
    using XF = typename std::conditional<KB == 32, h8_t, h4_t>::type;
    auto load_x = [&](int t, XF (&a)[NB]) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int k = t * SUBK + KB * b + (KB / 4) * mq;
            const uint32_t off = oob_unless((uint32_t)(((int64_t)mn * p.ldx + k) * 2), xkeep & (k < p.K ? 0xFFFFFFFFu : 0u));
            if constexpr (KB == 32) {
                a[b] = __builtin_bit_cast(h8_t, __builtin_amdgcn_raw_buffer_load_b128(xrs, off, 0, 0));
            } else {
                a[b] = __builtin_bit_cast(h4_t, __builtin_amdgcn_raw_buffer_load_b64(xrs, off, 0, 0));
            }
        }
    };

    f4_t acc = {0.f, 0.f, 0.f, 0.f};
    auto multiply = [&](const XF (&a)[NB]) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const float2 s = scl[scl_index<FMT>(b, mn)];
            const f4_t z = {0.f, 0.f, 0.f, 0.f};
            f4_t D, D2;
            if constexpr (KB == 32) {
                const h8_t B = *reinterpret_cast<const h8_t*>(bt + bt_unit<FMT>(b, mq, mn));
                D = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[b], B, z, 0, 0, 0);
                if constexpr (FMT == Q4_K) {
                    const h8_t one = {1, 1, 1, 1, 1, 1, 1, 1};
                    D2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[b], one, z, 0, 0, 0);
                }
            } else {
                const h4_t B = *reinterpret_cast<const h4_t*>(bt + bt_unit<FMT>(b, mq, mn));
                D = __builtin_amdgcn_mfma_f32_16x16x16f16(a[b], B, z, 0, 0, 0);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float v = fmaf(s.x, D[j], acc[j]);
                if constexpr (FMT == Q4_K) v = fmaf(-s.y, D2[j], v);
                acc[j] = v;
            }
        }
    };

    // this wave's sub-steps: wave, wave + kSplitK, ...; every wave runs the
    // same number of rounds, the sub-steps past K load nothing and add zero
    const int per_wave = (steps + kSplitK - 1) / kSplitK;
    const int rounds = (per_wave + DW - 1) / DW;
    auto sub = [&](int i) { return wave + kSplitK * i; };
    ChunkData<FMT> w[DW];
    XF xr[2][NB];
    load_x(sub(0), xr[0]);
    load_x(sub(1), xr[1]);
#pragma unroll
    for (int i = 0; i < DW; ++i) load_w(sub(i), w[i]);
    for (int r = 0; r < rounds; ++r) {
#pragma unroll
        for (int u = 0; u < DW; ++u) {
            const int i = r * DW + u;
            decode_to_tile<FMT>(w[u], ln, lj, bt, scl);
            asm volatile("" ::: "memory");  // the tile is read back under other types
            multiply(xr[u & 1]);
            asm volatile("" ::: "memory");  // and rewritten by the next sub-step
            load_w(sub(i + DW), w[u]);
            load_x(sub(i + 2), xr[u & 1]);
            // keep each sub-step's work together: without a barrier in the
            // loop the scheduler would otherwise interleave sub-steps and run
            // out of registers
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    red[wave * 64 + lane] = acc;
    __syncthreads();
    if (wave == 0) {
        f4_t t = red[lane];
#pragma unroll
        for (int v = 1; v < kSplitK; ++v) {
            const f4_t o = red[v * 64 + lane];
#pragma unroll
            for (int j = 0; j < 4; ++j) t[j] += o[j];
        }
        const int64_t row = row0 + mn;
        if (row < p.rows)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int m = 4 * mq + j;
                if (m < M) p.y[(int64_t)m * p.ldy + row] = t[j];
            }
    }
}

template <int FMT, int NT, bool XF32, int W>
static hipError_t launch_mfma_one(const MvParams& p, int M, uint32_t x_bytes, hipStream_t stream, hipEvent_t ev0,
                                  hipEvent_t ev1) {
    const size_t lds = MfmaLds<FMT, NT, XF32, W>::TOTAL;
    auto kernel = matvec_mfma<FMT, NT, XF32, W>;
    if (lds > 65536) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    const int64_t stripes = (p.rows + 15) / 16;
    const int grid = (int)((stripes + W - 1) / W);
    if (ev0 || ev1)
        hipExtLaunchKernelGGL(kernel, dim3(grid), dim3(64 * W), (uint32_t)lds, stream, ev0, ev1, 0u, p, M, x_bytes);
    else
        hipLaunchKernelGGL(kernel, dim3(grid), dim3(64 * W), lds, stream, p, M, x_bytes);
    return hipGetLastError();
}

// A single-wave workgroup stages all activations itself; it is kept to one
// 16-row tile of fp16 activations, where that fits in registers.
template <int NT, bool XF32>
constexpr int min_waves() {
    return NT == 1 && !XF32 ? 1 : 2;
}

template <int FMT, int NT, bool XF32>
static hipError_t launch_mfma_w(int W, const MvParams& p, int M, uint32_t x_bytes, hipStream_t stream, hipEvent_t ev0,
                                hipEvent_t ev1) {
    if (W == 4) return launch_mfma_one<FMT, NT, XF32, 4>(p, M, x_bytes, stream, ev0, ev1);
    if constexpr (min_waves<NT, XF32>() == 1)
        if (W == 1) return launch_mfma_one<FMT, NT, XF32, 1>(p, M, x_bytes, stream, ev0, ev1);
    return launch_mfma_one<FMT, NT, XF32, 2>(p, M, x_bytes, stream, ev0, ev1);
}

}  // namespace rq
