// Device-side decoders of one chunk of the repacked layout (layout.h).
//
// Integer form (dot_int, all quantized formats). Activations are staged per
// 32-value block b as 16-bit integers x = rint(v / s_b), s_b = max|v| / 30583,
// each split into four balanced hex digits x = sum_i 16^i d_i, d_i in [-8, 7],
// packed eight to a word in the weights' order (stage.h). A word of eight
// signed weight nibbles (q - 8) then dots with digit word i in one
// v_dot8_i32_i4, exactly in int32; the four digit sums are combined with
// shifts, and the block's scale and the format's scales are applied once per
// block in fp32:
//   Q4_0:  d * s_b * sum (q - 8) x
//   Q4_K:  d*sc * s_b * (sum (q - 8) x) + (8 d*sc - dmin*m) * s_b * sum x
//   Q8_0:  d * s_b * sum q x, with x split into two balanced bytes for v_dot4_i32_i8.
//   Q6_K:  d*sc * s_b * (sum q x - 32 sum x), q = l + 16 h assembled into bytes
//          (q6k_bytes), x as two balanced bytes, v_dot4_i32_i8: half the dot
//          instructions of a nibble form (which takes two per weight, one for
//          l and one for h, against four digits).
// The activation quantization is the only rounding beyond fp32 accumulation
// (relative 1/61166 of the block maximum per value).
//
// Exact form (decode_chunk): every weight decoded to its exact fp32 value in
// recipe's operation order (recipe.rs:3687-3833: d*sc*q - dmin*m for Q4_K,
// d*sc*(q-32) for Q6_K, (q-8)*d for Q4_0, q*d for Q8_0), used by the dequant
// kernel and the F16-weight path.
#pragma once

#include <hip/hip_runtime.h>

#include "layout.h"

namespace rq {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, a), __builtin_bit_cast(h2_t, b), c, false);
}
__device__ __forceinline__ int sdot8(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot8((int)a, (int)b, c, false);
}
__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

__device__ __forceinline__ uint32_t word(const uint4& v, int i) {
    return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}
__device__ __forceinline__ float wordf(const uint4& v, int i) { return __builtin_bit_cast(float, word(v, i)); }

__device__ __forceinline__ float half_lo(uint32_t v) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(v & 0xffffu));
}
__device__ __forceinline__ float half_hi(uint32_t v) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(v >> 16));
}

__device__ __forceinline__ uint32_t bfe(uint32_t v, uint32_t off, uint32_t width) {
    return __builtin_amdgcn_ubfe(v, off, width);
}
__device__ __forceinline__ int sbfe(uint32_t v, uint32_t off, uint32_t width) {
    return __builtin_amdgcn_sbfe((int)v, off, width);
}

// Per-format traits used by the generic kernels.
//   CW  weights per chunk          QP  16-byte code parts per chunk
//   XP  16-byte activation parts per chunk (digit words, or fp16 pairs for F16)
//   BLK 32-value activation blocks per chunk
//   XR  16-byte rows of staged block data per chunk (2 + one outlier row per block)
template <int FMT> struct Traits;
template <> struct Traits<Q8_0> { static constexpr int CW = 32, QP = 2, XP = 4, BLK = 1, XR = 3; };
template <> struct Traits<Q4_0> { static constexpr int CW = 64, QP = 2, XP = 8, BLK = 2, XR = 4; };
template <> struct Traits<Q4_K> { static constexpr int CW = 64, QP = 2, XP = 8, BLK = 2, XR = 4; };
template <> struct Traits<Q6_K> { static constexpr int CW = 64, QP = 3, XP = 8, BLK = 2, XR = 4; };
template <> struct Traits<F16> { static constexpr int CW = 64, QP = 8, XP = 8, BLK = 2, XR = 0; };

// One chunk's weight data as loaded from HBM.
template <int FMT> struct ChunkData {
    uint4 q[Traits<FMT>::QP];
    uint4 meta;  // meaning depends on the format (see load_chunk)
};

// A repacked weight as the kernels see it: rows of row_bytes (layout.h).
struct Planes {
    const uint8_t* base;
    int64_t row_bytes;
    int nch;         // chunks per row
    uint32_t bytes;  // bytes readable from base (buffer loads past them return zeros)
};

// Offset that every buffer load treats as out of range: such a load returns
// zeros and touches no memory. Weights are kept below it (the loader checks).
constexpr uint32_t kOobOffset = 0xFFFFFF00u;

// Bytes of a full 64-chunk group (layout.h group_bytes(64)).
template <int FMT>
constexpr uint32_t full_group_bytes() {
    return 64u * Traits<FMT>::QP * 16u + (FMT == Q8_0 ? 128u : FMT == Q6_K ? 288u : FMT == F16 ? 0u : 256u);
}

__device__ __forceinline__ uint4 ld16(const uint8_t* p) { return *reinterpret_cast<const uint4*>(p); }
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld16_nt(const uint8_t* p) {
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// Loads chunk c of physical row `row`. Offsets are 32-bit (a weight is smaller
// than 4 GiB, which the loader checks), so the loads take a scalar base
// address plus one VGPR offset each.
template <int FMT>
__device__ __forceinline__ void load_chunk(const Planes& P, int64_t row, int c, ChunkData<FMT>& d) {
    constexpr int QP = Traits<FMT>::QP;
    const uint32_t group = (uint32_t)c >> 6, within = (uint32_t)c & 63u;
    const uint32_t rest = (uint32_t)P.nch - (group << 6);
    const uint32_t nb = rest > 64u ? 64u : rest;
    const uint32_t gb = (uint32_t)row * (uint32_t)P.row_bytes + group * full_group_bytes<FMT>();
#pragma unroll
    for (int h = 0; h < QP; ++h) d.q[h] = ld16_nt(P.base + (gb + ((uint32_t)h * nb + within) * 16u));
    const uint32_t meta = gb + (uint32_t)QP * nb * 16u;
    if constexpr (FMT == Q4_K) {
        d.meta = ld16(P.base + (meta + (within >> 2) * 16u));
    } else if constexpr (FMT == Q6_K) {
        const uint32_t sc = *reinterpret_cast<const uint32_t*>(P.base + (meta + (within >> 2) * 16u + (within & 3u) * 4u));
        const uint16_t dd = *reinterpret_cast<const uint16_t*>(P.base + (meta + (nb >> 2) * 16u + (within >> 2) * 2u));
        d.meta = make_uint4(sc, dd, 0, 0);
    } else if constexpr (FMT == Q4_0) {
        d.meta = make_uint4(*reinterpret_cast<const uint32_t*>(P.base + (meta + within * 4u)), 0, 0, 0);
    } else if constexpr (FMT == Q8_0) {
        d.meta = make_uint4(*reinterpret_cast<const uint16_t*>(P.base + (meta + within * 2u)), 0, 0, 0);
    } else {
        d.meta = make_uint4(0, 0, 0, 0);
    }
}

// `off` where `keep` is all ones, kOobOffset where it is zero. Written as a
// bit select so that the compiler keeps one unconditional load instead of
// branching around it.
__device__ __forceinline__ uint32_t oob_unless(uint32_t off, uint32_t keep) {
    return (off & keep) | (kOobOffset & ~keep);
}

// Buffer resource over a weight's bytes: raw (stride 0) addressing with
// 32-bit data format, so a dword load at or past `bytes` returns zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t planes_rsrc(const Planes& P) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(P.base), (short)0, (int)P.bytes, 0x00020000);
}

// load_chunk through a buffer resource. A lane with `valid` false loads from
// kOobOffset: zeros, no memory traffic, and the same instruction count as
// every other lane, so the waits on earlier loads stay exact.
template <int FMT>
__device__ __forceinline__ void load_chunk_rs(__amdgpu_buffer_rsrc_t rs, const Planes& P, uint32_t row, int c, bool valid,
                                              ChunkData<FMT>& d) {
    constexpr int QP = Traits<FMT>::QP;
    const uint32_t group = (uint32_t)c >> 6, within = (uint32_t)c & 63u;
    const uint32_t rest = (uint32_t)P.nch - (group << 6);
    const uint32_t nb = rest > 64u ? 64u : rest;
    const uint32_t gb = row * (uint32_t)P.row_bytes + group * full_group_bytes<FMT>();
    const uint32_t keep = valid ? 0xFFFFFFFFu : 0u;
    auto at = [&](uint32_t off) { return oob_unless(off, keep); };
#pragma unroll
    for (int h = 0; h < QP; ++h) {
        const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rs, at(gb + ((uint32_t)h * nb + within) * 16u), 0, 0);
        d.q[h] = make_uint4(v.x, v.y, v.z, v.w);
    }
    const uint32_t meta = gb + (uint32_t)QP * nb * 16u;
    if constexpr (FMT == Q4_K) {
        const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rs, at(meta + (within >> 2) * 16u), 0, 0);
        d.meta = make_uint4(v.x, v.y, v.z, v.w);
    } else if constexpr (FMT == Q6_K) {
        const uint32_t sc = __builtin_amdgcn_raw_buffer_load_b32(rs, at(meta + (within >> 2) * 16u + (within & 3u) * 4u), 0, 0);
        const uint32_t dd = __builtin_amdgcn_raw_buffer_load_b16(rs, at(meta + (nb >> 2) * 16u + (within >> 2) * 2u), 0, 0);
        d.meta = make_uint4(sc, dd, 0, 0);
    } else if constexpr (FMT == Q4_0) {
        d.meta = make_uint4(__builtin_amdgcn_raw_buffer_load_b32(rs, at(meta + within * 4u), 0, 0), 0, 0, 0);
    } else if constexpr (FMT == Q8_0) {
        d.meta = make_uint4(__builtin_amdgcn_raw_buffer_load_b16(rs, at(meta + within * 2u), 0, 0), 0, 0, 0);
    } else {
        d.meta = make_uint4(0, 0, 0, 0);
    }
}

// Q4_K scale/min of the two sub-blocks 2p and 2p+1 of a chunk, from the
// superblock's meta words (x = d, dmin; y, z, w = the 96-bit scale fields):
// chunk p's 24-bit field at bit 24p holds scale(2p), min(2p), scale(2p+1),
// min(2p+1), six bits each (the repack's form of the k_scale bytes,
// recipe.rs:15204-15210). A 64-bit shift of (z:y) or (w:z) brings the field
// to bit 0: a selection between those pairs, as in word_at (a run-time choice
// between meta's members reads as an index into the register array, which
// the compiler would place in scratch memory).
__device__ __forceinline__ uint32_t q4k_field(const uint4& meta, int p) {
    const uint64_t lo = ((uint64_t)meta.z << 32) | meta.y, hi = ((uint64_t)meta.w << 32) | meta.z;
    const uint32_t sh = (uint32_t)(24 * p) - (p < 2 ? 0u : 32u);  // 0, 24, 16, 40
    return (uint32_t)((p < 2 ? lo : hi) >> sh);
}
__device__ __forceinline__ void q4k_scales(const uint4& meta, int p, uint32_t& sc0, uint32_t& m0, uint32_t& sc1,
                                           uint32_t& m1) {
    const uint32_t f = q4k_field(meta, p);
    sc0 = f & 63u;
    m0 = bfe(f, 6, 6);
    sc1 = bfe(f, 12, 6);
    m1 = bfe(f, 18, 6);
}

// sum_i 16^i sum_w dot8(W_w, D_i,w) over four weight words and the four digit
// words of each digit (digit i's words are xd[2i + half]), as one chain from
// digit 3 down (the running sum times 16 before each digit's dots): no
// accumulator starts from zero but the first, and no partial sums are combined
// afterwards. The sum is exact (|x| <= 30583, |q - 8| <= 8: below 2^24).
__device__ __forceinline__ int dot_nibbles4(const uint4& W, const uint4* xd, int half) {
    int t = 0;
#pragma unroll
    for (int i = 3; i >= 0; --i) {
        const uint4 D = xd[2 * i + half];
        t = sdot8(W.x, D.x, t * 16);
        t = sdot8(W.y, D.y, t);
        t = sdot8(W.z, D.z, t);
        t = sdot8(W.w, D.w, t);
    }
    return t;
}

// -------------------------------------------------------------------------
// Integer dot of one chunk for one activation row. xd[] holds the chunk's
// activation digit words as staged (Traits::XP parts), xb[] its block data:
// xb[0] = (s_0, s_1, sx_0, sx_1), xb[1] = (sx_2, sx_3, idx_0, idx_1), where s_b is
// block b's scale (its sign bit set when the block has extracted values) and sx
// the scaled activation sums (per 32-block for Q4_K, per 16-value scale group
// for Q6_K). Accumulates sum_j w_j x_j into acc, the outliers' terms aside
// (dot_outliers).
// -------------------------------------------------------------------------

// Word i (0..3, per lane) of a 16-byte part, by selects and a shift (a
// run-time index into the registers would go through scratch memory).
__device__ __forceinline__ uint32_t word_at(const uint4& v, int i) {
    const uint64_t lo = ((uint64_t)v.y << 32) | v.x, hi = ((uint64_t)v.w << 32) | v.z;
    const uint64_t pair = (i & 2) ? hi : lo;
    return (uint32_t)(pair >> (32 * (i & 1)));
}

// The 6-bit codes q = l + 16 h of 16-weight scale group g of a Q6_K chunk as
// four words of four bytes: the group's weights 0, 2, 4, 6 | 1, 3, 5, 7 |
// 8, 10, 12, 14 | 9, 11, 13, 15 (the staged activations' byte order). The low
// nibbles come un-XORed from the two code words of the group (weight 2j in the
// low nibble of byte j); h of weight j sits at bits 4j and of weight 8 + j at
// bits 4j + 2 of the group's high-field word, so shifts of it by 4, 0, 2 and
// -2 bring the four words' fields to bits 4-5 of their bytes. Plain shifts,
// ands and ors (on gfx950 each issues in about 0.6 of the time of a bit-field
// extract, a byte permute or a three-input logic op).
__device__ __forceinline__ void q6k_bytes(const ChunkData<Q6_K>& d, int g, uint32_t (&W)[4]) {
    const uint32_t L0 = word(d.q[g >> 1], (g & 1) * 2) ^ 0x88888888u;
    const uint32_t L1 = word(d.q[g >> 1], (g & 1) * 2 + 1) ^ 0x88888888u;
    const uint32_t H = word(d.q[2], g);
    W[0] = (L0 & 0x0F0F0F0Fu) | ((H << 4) & 0x30303030u);
    W[1] = ((L0 >> 4) & 0x0F0F0F0Fu) | (H & 0x30303030u);
    W[2] = (L1 & 0x0F0F0F0Fu) | ((H << 2) & 0x30303030u);
    W[3] = ((L1 >> 4) & 0x0F0F0F0Fu) | ((H >> 2) & 0x30303030u);
}

// True in every active lane when the chunk of any active lane holds an outlier.
__device__ __forceinline__ bool wave_has_outlier(const uint4& b0) {
    return __builtin_amdgcn_ballot_w64(((b0.x | b0.y) >> 31) != 0) != 0;
}

// Words of a chunk that every activation row's dot reads again: Q6_K's byte
// words (q6k_bytes, formed once per chunk however many rows it meets); the
// other formats dot their code words as loaded.
template <int FMT>
struct ChunkWords {
    uint32_t w[FMT == Q6_K ? 16 : 1];
};
template <int FMT>
__device__ __forceinline__ void chunk_words(const ChunkData<FMT>& d, ChunkWords<FMT>& cw) {
    if constexpr (FMT == Q6_K) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            uint32_t W[4];
            q6k_bytes(d, g, W);
#pragma unroll
            for (int i = 0; i < 4; ++i) cw.w[4 * g + i] = W[i];
        }
    }
}

template <int FMT>
__device__ __forceinline__ void dot_int_w(const ChunkData<FMT>& d, const ChunkWords<FMT>& cw, int c,
                                          const uint4 (&xd)[Traits<FMT>::XP], const uint4 (&xb)[2], float& acc) {
    const float sb0 = fabsf(wordf(xb[0], 0)), sb1 = fabsf(wordf(xb[0], 1));
    if constexpr (FMT == Q4_K) {
        uint32_t sc0, m0, sc1, m1;
        q4k_scales(d.meta, c & 3, sc0, m0, sc1, m1);
        const float dd = half_lo(d.meta.x), dmin = half_hi(d.meta.x);
        const float s0 = dd * (float)sc0, s1 = dd * (float)sc1;
        const float k0 = fmaf(8.f, s0, -dmin * (float)m0), k1 = fmaf(8.f, s1, -dmin * (float)m1);
        const int a0 = dot_nibbles4(d.q[0], xd, 0);
        const int a1 = dot_nibbles4(d.q[1], xd, 1);
        float y = acc;
        y = fmaf(s0 * sb0, (float)a0, y);
        y = fmaf(k0, wordf(xb[0], 2), y);
        y = fmaf(s1 * sb1, (float)a1, y);
        y = fmaf(k1, wordf(xb[0], 3), y);
        acc = y;
    } else if constexpr (FMT == Q4_0) {
        const float d0 = half_lo(d.meta.x), d1 = half_hi(d.meta.x);
        const int a0 = dot_nibbles4(d.q[0], xd, 0);
        const int a1 = dot_nibbles4(d.q[1], xd, 1);
        float y = acc;
        y = fmaf(d0 * sb0, (float)a0, y);
        y = fmaf(d1 * sb1, (float)a1, y);
        acc = y;
    } else if constexpr (FMT == Q8_0) {
        const float dd = half_lo(d.meta.x);
        // digit planes: xd[0..1] low bytes, xd[2..3] high bytes (words 0-3,
        // 4-7); the high bytes' sum times 256, then the low bytes' dots, in
        // one chain (exact: |sum q x| <= 32 * 128 * 30583 < 2^31)
        int t = 0;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint4 W = d.q[h], H = xd[2 + h];
            t = sdot4(W.x, H.x, t);
            t = sdot4(W.y, H.y, t);
            t = sdot4(W.z, H.z, t);
            t = sdot4(W.w, H.w, t);
        }
        t *= 256;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint4 W = d.q[h], L = xd[h];
            t = sdot4(W.x, L.x, t);
            t = sdot4(W.y, L.y, t);
            t = sdot4(W.z, L.z, t);
            t = sdot4(W.w, L.w, t);
        }
        acc = fmaf(dd * sb0, (float)t, acc);
    } else if constexpr (FMT == Q6_K) {
        const float dd = half_lo(d.meta.y);
        float y = acc;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const uint32_t* W = cw.w + 4 * g;
            const float dsc = dd * (float)(int8_t)((d.meta.x >> (8 * g)) & 0xffu);
            // the high bytes' sum times 256, then the low bytes' dots, in one
            // chain (exact: |sum q x| <= 16 * 63 * 30583 < 2^31)
            const uint4 Lo = xd[g], Hi = xd[4 + g];
            int t = sdot4(W[0], Hi.x, 0);
            t = sdot4(W[1], Hi.y, t);
            t = sdot4(W[2], Hi.z, t);
            t = sdot4(W[3], Hi.w, t);
            t *= 256;
            t = sdot4(W[0], Lo.x, t);
            t = sdot4(W[1], Lo.y, t);
            t = sdot4(W[2], Lo.z, t);
            t = sdot4(W[3], Lo.w, t);
            const float s = g < 2 ? sb0 : sb1;
            const float sx = g < 2 ? wordf(xb[0], 2 + g) : wordf(xb[1], g - 2);
            y = fmaf(dsc * s, (float)t, y);
            y = fmaf(-32.f * dsc, sx, y);
        }
        acc = y;
    }
}

template <int FMT>
__device__ __forceinline__ void dot_int(const ChunkData<FMT>& d, int c, const uint4 (&xd)[Traits<FMT>::XP],
                                        const uint4 (&xb)[2], float& acc) {
    ChunkWords<FMT> cw;
    chunk_words<FMT>(d, cw);
    dot_int_w<FMT>(d, cw, c, xd, xb, acc);
}

// The extracted activations' terms of one chunk. `xo` points at the chunk's
// staged block data (row 0 of its XR rows, `nch` 16-byte units apart): row 1
// holds in words 2 + b the slot indices of block b (five bits per slot, slot j
// at bits 5j), row 2 + b block b's four slot values (0 in unused slots). Adds
// w_i v for every slot, with the weight decoded exactly (w = d sc q - dmin m
// for Q4_K, d (q - 8) for Q4_0, d q for Q8_0, d sc (q - 32) for Q6_K). Run
// when wave_has_outlier says some lane of the wave needs it.
template <int FMT>
__device__ __forceinline__ void dot_outliers(const ChunkData<FMT>& d, int c, const uint4* xo, int nch, float& acc) {
    constexpr int BLK = Traits<FMT>::BLK;
    const uint4 ix = xo[nch];
    float y = acc;
    float sc[2], k[2] = {0.f, 0.f};
    if constexpr (FMT == Q4_K) {
        uint32_t sc0, m0, sc1, m1;
        q4k_scales(d.meta, c & 3, sc0, m0, sc1, m1);
        const float dd = half_lo(d.meta.x), dmin = half_hi(d.meta.x);
        sc[0] = dd * (float)sc0;
        sc[1] = dd * (float)sc1;
        k[0] = fmaf(8.f, sc[0], -dmin * (float)m0);
        k[1] = fmaf(8.f, sc[1], -dmin * (float)m1);
    } else if constexpr (FMT == Q4_0) {
        sc[0] = half_lo(d.meta.x);
        sc[1] = half_hi(d.meta.x);
    }
#pragma unroll
    for (int b = 0; b < BLK; ++b) {
        const uint4 ov = xo[(2 + b) * nch];
        const uint32_t idx = word(ix, 2 + b);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int i = (int)bfe(idx, 5 * j, 5);
            const float v = wordf(ov, j);
            if constexpr (FMT == Q4_K) {
                const int q = sbfe(word_at(d.q[b], i >> 3), 4 * (i & 7), 4);
                y = fmaf(fmaf(sc[b], (float)q, k[b]), v, y);
            } else if constexpr (FMT == Q4_0) {
                const int q = sbfe(word_at(d.q[b], i >> 3), 4 * (i & 7), 4);
                y = fmaf((float)q * sc[b], v, y);
            } else if constexpr (FMT == Q8_0) {
                const uint32_t w0 = word_at(d.q[0], (i >> 2) & 3), w1 = word_at(d.q[1], (i >> 2) & 3);
                const uint32_t wd = i < 16 ? w0 : w1;  // (selecting the part first would index registers at run time)
                y = fmaf(half_lo(d.meta.x) * (float)sbfe(wd, 8 * (i & 3), 8), v, y);
            } else if constexpr (FMT == Q6_K) {
                // position e = 32 b + i of the chunk, in scale group e / 16
                const int e = 32 * b + i, g = e >> 4, jj = e & 15;
                const int l = sbfe(word_at(d.q[b], (e >> 3) & 3), 4 * (e & 7), 4) + 8;
                const int h = (int)bfe(word_at(d.q[2], g), jj < 8 ? 4 * jj : 4 * (jj - 8) + 2, 2);
                const float dsc = half_lo(d.meta.y) * (float)(int8_t)((d.meta.x >> (8 * g)) & 0xffu);
                y = fmaf(dsc * (float)(l + 16 * h - 32), v, y);
            }
        }
    }
    acc = y;
}

// fp16 activation pairs against F16 weights (router-sized products).
template <int M>
__device__ __forceinline__ void dot_f16w(const ChunkData<F16>& d, const uint4 (*xp)[8], float* acc) {
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
            const int q0 = sbfe(word(d.q[0], i >> 3), 4 * (i & 7), 4) + 8;
            const int q1 = sbfe(word(d.q[1], i >> 3), 4 * (i & 7), 4) + 8;
            out[i] = fmaf(s0, (float)q0, -n0);
            out[32 + i] = fmaf(s1, (float)q1, -n1);
        }
    } else if constexpr (FMT == Q4_0) {
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
            const float dd = blk ? half_hi(d.meta.x) : half_lo(d.meta.x);
#pragma unroll
            for (int i = 0; i < 32; ++i) out[32 * blk + i] = (float)sbfe(word(d.q[blk], i >> 3), 4 * (i & 7), 4) * dd;
        }
    } else if constexpr (FMT == Q8_0) {
        const float dd = half_lo(d.meta.x);
#pragma unroll
        for (int i = 0; i < 32; ++i) out[i] = (float)sbfe(word(d.q[i >> 4], (i >> 2) & 3), 8 * (i & 3), 8) * dd;
    } else if constexpr (FMT == Q6_K) {
        const float dd = half_lo(d.meta.y);
#pragma unroll
        for (int e = 0; e < 64; ++e) {
            const int g = e >> 4, j = e & 15;
            const int l = sbfe(word(d.q[e >> 5], (e >> 3) & 3), 4 * (e & 7), 4) + 8;
            const int h = (int)bfe(word(d.q[2], g), j < 8 ? 4 * j : 4 * (j - 8) + 2, 2);
            const float dsc = dd * (float)(int8_t)((d.meta.x >> (8 * g)) & 0xffu);
            out[e] = dsc * (float)(l + 16 * h - 32);
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
