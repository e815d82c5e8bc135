// Device-side decoders of one chunk of the repacked layout (layout.h).
//
// Two arithmetic forms:
//  * dot_f16: activations are fp16. Codes are turned into fp16 pairs with one
//    mask-and-or each, 1024 + q or 1024 + 16 q (0x6400 is 1024.0 in binary16
//    and a code of up to 10 bits fills its mantissa exactly), and dotted with
//    v_dot2_f32_f16 into fp32. The 1024 offsets and the format's constant code
//    offset (Q4_0's 8, Q6_K's 32, Q8_0's 128 bias) are removed per scale group
//    with sums of the activations, and the per-group scales are applied once
//    per group: sum_j (s q_j - m) x_j = s * sum_j q_j x_j - m * sum_j x_j.
//  * dot_f32 / decode: every weight is decoded to its exact fp32 value, in the
//    same operation order as recipe's dequantization (recipe.rs:3687-3833:
//    d*sc*q - dmin*m for Q4_K, d*sc*(q-32) for Q6_K, (q-8)*d for Q4_0, q*d for
//    Q8_0), then fma'd with fp32 activations.
#pragma once

#include <hip/hip_runtime.h>

#include "layout.h"

namespace rq {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, a), __builtin_bit_cast(h2_t, b), c, false);
}

__device__ __forceinline__ uint32_t word(const uint4& v, int i) {
    return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}

__device__ __forceinline__ float half_lo(uint32_t v) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(v & 0xffffu));
}
__device__ __forceinline__ float half_hi(uint32_t v) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(v >> 16));
}

__device__ __forceinline__ uint32_t bfe(uint32_t v, uint32_t off, uint32_t width) {
    return __builtin_amdgcn_ubfe(v, off, width);
}

__device__ __forceinline__ uint32_t rotr(uint32_t v, uint32_t s) { return __builtin_amdgcn_alignbit(v, v, s); }

constexpr uint32_t kMagic = 0x64006400u;  // two binary16 1024.0

// Per-format traits used by the generic kernels.
template <int FMT> struct Traits;
template <> struct Traits<Q8_0> { static constexpr int CW = 32, QP = 2, NS = 1, PERM4 = 1; };
template <> struct Traits<Q4_0> { static constexpr int CW = 64, QP = 2, NS = 4, PERM4 = 1; };
template <> struct Traits<Q4_K> { static constexpr int CW = 64, QP = 2, NS = 2, PERM4 = 1; };
template <> struct Traits<Q6_K> { static constexpr int CW = 64, QP = 3, NS = 8, PERM4 = 0; };
template <> struct Traits<F16> { static constexpr int CW = 64, QP = 8, NS = 0, PERM4 = 0; };

// One chunk's weight data as loaded from HBM.
template <int FMT> struct ChunkData {
    uint4 q[Traits<FMT>::QP];
    uint4 meta;  // meaning depends on the format (see load_chunk)
};

struct Planes {
    const uint8_t* code;
    const uint8_t* meta0;
    const uint8_t* meta1;
    int64_t row_code, row_meta0, row_meta1;  // bytes per row in each plane
    int nch;                                 // chunks per row
};

__device__ __forceinline__ uint4 ld16(const uint8_t* p) { return *reinterpret_cast<const uint4*>(p); }
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld16_nt(const uint8_t* p) {
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// Loads chunk c of physical row `row`.
template <int FMT>
__device__ __forceinline__ void load_chunk(const Planes& P, int64_t row, int c, ChunkData<FMT>& d) {
    constexpr int QP = Traits<FMT>::QP;
    const uint8_t* cr = P.code + row * P.row_code;
#pragma unroll
    for (int h = 0; h < QP; ++h) d.q[h] = ld16_nt(cr + code_offset(c, h, P.nch, QP));
    if constexpr (FMT == Q4_K) {
        d.meta = ld16(P.meta0 + row * P.row_meta0 + (int64_t)(c >> 2) * 16);
    } else if constexpr (FMT == Q6_K) {
        const uint32_t sc = *reinterpret_cast<const uint32_t*>(P.meta0 + row * P.row_meta0 + (int64_t)(c >> 2) * 16 + (c & 3) * 4);
        const uint16_t dd = *reinterpret_cast<const uint16_t*>(P.meta1 + row * P.row_meta1 + (int64_t)(c >> 2) * 2);
        d.meta = make_uint4(sc, dd, 0, 0);
    } else if constexpr (FMT == Q4_0) {
        d.meta = make_uint4(*reinterpret_cast<const uint32_t*>(P.meta0 + row * P.row_meta0 + (int64_t)c * 4), 0, 0, 0);
    } else if constexpr (FMT == Q8_0) {
        d.meta = make_uint4(*reinterpret_cast<const uint16_t*>(P.meta0 + row * P.row_meta0 + (int64_t)c * 2), 0, 0, 0);
    } else {
        d.meta = make_uint4(0, 0, 0, 0);
    }
}

// Q4_K scale/min of the two sub-blocks 2p and 2p+1 of a chunk, from the
// superblock's 12 scale bytes s[] held as words m1 = s[0..3], m2 = s[4..7],
// m3 = s[8..11]; the k_scale packing of recipe.rs:15204-15210.
__device__ __forceinline__ void q4k_scales(const uint4& meta, int p, uint32_t& sc0, uint32_t& m0, uint32_t& sc1,
                                           uint32_t& m1) {
    const uint32_t o = 16u * (uint32_t)(p & 1);
    const bool hi = p >= 2;
    const uint32_t X = hi ? meta.w : meta.y;  // low 4 bits of the scale
    const uint32_t Y = hi ? meta.w : meta.z;  // low 4 bits of the minimum
    const uint32_t xo = 0, yo = hi ? 4u : 0u;
    const uint32_t top = hi ? 6u : 4u;
    sc0 = bfe(X, o + xo, 4) | (bfe(meta.y, o + top, 2) << 4);
    sc1 = bfe(X, o + 8 + xo, 4) | (bfe(meta.y, o + 8 + top, 2) << 4);
    m0 = bfe(Y, o + yo, 4) | (bfe(meta.z, o + top, 2) << 4);
    m1 = bfe(Y, o + 8 + yo, 4) | (bfe(meta.z, o + 8 + top, 2) << 4);
}

// -------------------------------------------------------------------------
// fp16 activations. xp[] holds the chunk's activation pairs as laid out in
// LDS (Traits::PERM4: each run of four values a,b,c,d stored a,c,b,d), s[] the
// chunk's activation sums. Accumulates sum_j w_j x_j into acc.
// -------------------------------------------------------------------------
template <int FMT, int M>
__device__ __forceinline__ void dot_f16(const ChunkData<FMT>& d, int c, const uint4 (*xp)[Traits<FMT>::CW / 8],
                                        const float (*s)[Traits<FMT>::NS > 0 ? Traits<FMT>::NS : 1], float* acc) {
    if constexpr (FMT == Q4_K) {
        float alo[M], ahi[M];
#pragma unroll
        for (int m = 0; m < M; ++m) alo[m] = ahi[m] = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t w = word(d.q[i >> 2], i & 3);
            const uint32_t w8 = w >> 8;
            const uint32_t a = (w & 0x000F000Fu) | kMagic, cc = (w8 & 0x000F000Fu) | kMagic;
            const uint32_t b = (w & 0x00F000F0u) | kMagic, e = (w8 & 0x00F000F0u) | kMagic;
#pragma unroll
            for (int m = 0; m < M; ++m) {
                alo[m] = dot2(a, word(xp[m][i >> 1], (i & 1) * 2), alo[m]);
                alo[m] = dot2(cc, word(xp[m][i >> 1], (i & 1) * 2 + 1), alo[m]);
                ahi[m] = dot2(b, word(xp[m][4 + (i >> 1)], (i & 1) * 2), ahi[m]);
                ahi[m] = dot2(e, word(xp[m][4 + (i >> 1)], (i & 1) * 2 + 1), ahi[m]);
            }
        }
        uint32_t sc0, m0, sc1, m1;
        q4k_scales(d.meta, c & 3, sc0, m0, sc1, m1);
        const float dd = half_lo(d.meta.x), dmin = half_hi(d.meta.x);
        const float s0 = dd * (float)sc0, s1 = dd * (float)sc1;
        const float n0 = dmin * (float)m0, n1 = dmin * (float)m1;
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const float tlo = fmaf(-1024.f, s[m][0], alo[m]);
            const float thi = fmaf(-64.f, s[m][1], ahi[m] * 0.0625f);
            float y = acc[m];
            y = fmaf(s0, tlo, y);
            y = fmaf(-n0, s[m][0], y);
            y = fmaf(s1, thi, y);
            y = fmaf(-n1, s[m][1], y);
            acc[m] = y;
        }
    } else if constexpr (FMT == Q4_0) {
        const float d0 = half_lo(d.meta.x), d1 = half_hi(d.meta.x);
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
            float a1[M], a16[M];
#pragma unroll
            for (int m = 0; m < M; ++m) a1[m] = a16[m] = 0.f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t w = word(d.q[blk], i);
                const uint32_t w8 = w >> 8;
                const uint32_t a = (w & 0x000F000Fu) | kMagic, cc = (w8 & 0x000F000Fu) | kMagic;
                const uint32_t b = (w & 0x00F000F0u) | kMagic, e = (w8 & 0x00F000F0u) | kMagic;
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    const uint4 xl = xp[m][4 * blk + (i >> 1)];
                    const uint4 xh = xp[m][4 * blk + 2 + (i >> 1)];
                    a1[m] = dot2(a, word(xl, (i & 1) * 2), a1[m]);
                    a1[m] = dot2(cc, word(xl, (i & 1) * 2 + 1), a1[m]);
                    a16[m] = dot2(b, word(xh, (i & 1) * 2), a16[m]);
                    a16[m] = dot2(e, word(xh, (i & 1) * 2 + 1), a16[m]);
                }
            }
            const float db = blk ? d1 : d0;
#pragma unroll
            for (int m = 0; m < M; ++m) {
                float t = fmaf(a16[m], 0.0625f, a1[m]);
                t = fmaf(-1032.f, s[m][2 * blk], t);
                t = fmaf(-72.f, s[m][2 * blk + 1], t);
                acc[m] = fmaf(db, t, acc[m]);
            }
        }
    } else if constexpr (FMT == Q8_0) {
        float a[M];
#pragma unroll
        for (int m = 0; m < M; ++m) a[m] = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t w = word(d.q[i >> 2], i & 3);
            const uint32_t lo = (w & 0x00FF00FFu) | kMagic, hi = ((w >> 8) & 0x00FF00FFu) | kMagic;
#pragma unroll
            for (int m = 0; m < M; ++m) {
                a[m] = dot2(lo, word(xp[m][i >> 1], (i & 1) * 2), a[m]);
                a[m] = dot2(hi, word(xp[m][i >> 1], (i & 1) * 2 + 1), a[m]);
            }
        }
        const float dd = half_lo(d.meta.x);
#pragma unroll
        for (int m = 0; m < M; ++m) acc[m] = fmaf(dd, fmaf(-1152.f, s[m][0], a[m]), acc[m]);
    } else if constexpr (FMT == Q6_K) {
        const float dd = half_lo(d.meta.y);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const uint32_t A = word(d.q[g >> 1], (g & 1) * 2), B = word(d.q[g >> 1], (g & 1) * 2 + 1);
            const uint32_t H = word(d.q[2], g);
            const uint32_t A8 = A >> 8, B8 = B >> 8, H2 = H >> 2, R8 = rotr(H, 8), R10 = rotr(H, 10);
            const uint32_t p0 = (A & 0x000F000Fu) | (H & 0x00300030u) | kMagic;
            const uint32_t p2 = (A8 & 0x000F000Fu) | (H2 & 0x00300030u) | kMagic;
            const uint32_t p4 = (B & 0x000F000Fu) | (R8 & 0x00300030u) | kMagic;
            const uint32_t p6 = (B8 & 0x000F000Fu) | (R10 & 0x00300030u) | kMagic;
            const uint32_t p8 = (A & 0x00F000F0u) | (H & 0x03000300u) | kMagic;
            const uint32_t p10 = (A8 & 0x00F000F0u) | (H2 & 0x03000300u) | kMagic;
            const uint32_t p12 = (B & 0x00F000F0u) | (R8 & 0x03000300u) | kMagic;
            const uint32_t p14 = (B8 & 0x00F000F0u) | (R10 & 0x03000300u) | kMagic;
            const float sc = dd * (float)(int8_t)((d.meta.x >> (8 * g)) & 0xffu);
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const uint4 x0 = xp[m][2 * g], x1 = xp[m][2 * g + 1];
                float a1 = dot2(p0, x0.x, 0.f);
                a1 = dot2(p2, x0.y, a1);
                a1 = dot2(p4, x0.z, a1);
                a1 = dot2(p6, x0.w, a1);
                float a16 = dot2(p8, x1.x, 0.f);
                a16 = dot2(p10, x1.y, a16);
                a16 = dot2(p12, x1.z, a16);
                a16 = dot2(p14, x1.w, a16);
                float t = fmaf(a16, 0.0625f, a1);
                t = fmaf(-1056.f, s[m][2 * g], t);
                t = fmaf(-96.f, s[m][2 * g + 1], t);
                acc[m] = fmaf(sc, t, acc[m]);
            }
        }
    } else if constexpr (FMT == F16) {
#pragma unroll
        for (int m = 0; m < M; ++m) {
            float a = acc[m];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                a = dot2(d.q[j].x, xp[m][j].x, a);
                a = dot2(d.q[j].y, xp[m][j].y, a);
                a = dot2(d.q[j].z, xp[m][j].z, a);
                a = dot2(d.q[j].w, xp[m][j].w, a);
            }
            acc[m] = a;
        }
    }
}

// -------------------------------------------------------------------------
// Exact fp32 decode of a chunk: out[v] for v = 0..CW-1 in natural (GGUF)
// order within the chunk.
// -------------------------------------------------------------------------
template <int FMT>
__device__ __forceinline__ void decode_chunk(const ChunkData<FMT>& d, int c, float* out) {
    if constexpr (FMT == Q4_K) {
        uint32_t sc0, m0, sc1, m1;
        q4k_scales(d.meta, c & 3, sc0, m0, sc1, m1);
        const float dd = half_lo(d.meta.x), dmin = half_hi(d.meta.x);
        const float s0 = dd * (float)sc0, s1 = dd * (float)sc1;
        const float n0 = dmin * (float)m0, n1 = dmin * (float)m1;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            const uint32_t byte = (word(d.q[i >> 4], (i >> 2) & 3) >> (8 * (i & 3))) & 0xffu;
            out[i] = fmaf(s0, (float)(byte & 15u), -n0);
            out[32 + i] = fmaf(s1, (float)(byte >> 4), -n1);
        }
    } else if constexpr (FMT == Q4_0) {
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
            const float dd = blk ? half_hi(d.meta.x) : half_lo(d.meta.x);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const uint32_t byte = (word(d.q[blk], i >> 2) >> (8 * (i & 3))) & 0xffu;
                out[32 * blk + i] = (float)((int)(byte & 15u) - 8) * dd;
                out[32 * blk + 16 + i] = (float)((int)(byte >> 4) - 8) * dd;
            }
        }
    } else if constexpr (FMT == Q8_0) {
        const float dd = half_lo(d.meta.x);
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            const uint32_t byte = (word(d.q[i >> 4], (i >> 2) & 3) >> (8 * (i & 3))) & 0xffu;
            out[i] = (float)((int)byte - 128) * dd;
        }
    } else if constexpr (FMT == Q6_K) {
        const float dd = half_lo(d.meta.y);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const uint32_t A = word(d.q[g >> 1], (g & 1) * 2), B = word(d.q[g >> 1], (g & 1) * 2 + 1);
            const uint32_t H = word(d.q[2], g);
            const uint32_t A8 = A >> 8, B8 = B >> 8, H2 = H >> 2, R8 = rotr(H, 8), R10 = rotr(H, 10);
            const uint32_t p[8] = {
                (A & 0x000F000Fu) | (H & 0x00300030u) | kMagic,   (A8 & 0x000F000Fu) | (H2 & 0x00300030u) | kMagic,
                (B & 0x000F000Fu) | (R8 & 0x00300030u) | kMagic,  (B8 & 0x000F000Fu) | (R10 & 0x00300030u) | kMagic,
                (A & 0x00F000F0u) | (H & 0x03000300u) | kMagic,   (A8 & 0x00F000F0u) | (H2 & 0x03000300u) | kMagic,
                (B & 0x00F000F0u) | (R8 & 0x03000300u) | kMagic,  (B8 & 0x00F000F0u) | (R10 & 0x03000300u) | kMagic};
            const float sc = dd * (float)(int8_t)((d.meta.x >> (8 * g)) & 0xffu);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                // 1024 + q (j < 4) or 1024 + 16 q (j >= 4), exact in fp16 and fp32.
                float lo = half_lo(p[j]) - 1024.f, hi = half_hi(p[j]) - 1024.f;
                if (j >= 4) {
                    lo *= 0.0625f;
                    hi *= 0.0625f;
                }
                out[16 * g + 2 * j] = sc * (lo - 32.f);
                out[16 * g + 2 * j + 1] = sc * (hi - 32.f);
            }
        }
    } else if constexpr (FMT == F16) {
#pragma unroll
        for (int j = 0; j < 32; ++j) {
            const uint32_t v = word(d.q[j >> 2], j & 3);
            out[2 * j] = half_lo(v);
            out[2 * j + 1] = half_hi(v);
        }
    }
}

}  // namespace rq
