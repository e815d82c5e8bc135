// Activation staging into LDS, shared by the matvec and MoE kernels.
//
// Quantized weights (integer kernels). Each 32-value block b of an activation
// row becomes 16-bit integers x = rint(v / s_b) with scale s_b = amax / 30583,
// amax the largest magnitude of the values the block encodes, so every such
// value is within s_b / 2 (1.64e-5 of amax) of s_b x. Large values are taken
// out first: when at most kOutlierSlots values of a block are at or above
// amax / kOutlierRatio, they go to the block's slots (encoded as 0) and the
// kernels multiply them exactly in fp32 with their weights; the test repeats
// on the rest with its own largest magnitude until the slots are used up or
// the rest has more large values than slots are left. So a block's step is at
// most kOutlierRatio / 30583 of its (kOutlierSlots + 1)-th largest magnitude:
// a few outliers per block (on columns whose weights are small or zero) do not
// coarsen the block's other values. For 4-bit formats each x is split into
// four balanced hex digits (x + 0x8888 has hex digits d_i + 8, so
// (x + 0x8888) ^ 0x8888 holds every d_i as a signed nibble) and the digits are
// transposed into words of eight values per digit, the weights' nibble order.
// For Q8_0 and Q6_K x is split into two balanced bytes ((x + 0x8080) ^ 0x8080)
// and transposed into words of four (Q6_K: the even and the odd values of
// eight, the order of its byte words).
//   LDS: xd [m][part][chunk] 16-byte digit words (Traits::XP parts per chunk:
//        Q4_0 and Q4_K: part 2i + b holds digit i of the chunk's block b;
//        Q8_0: parts 0-1 low bytes, parts 2-3 high bytes; Q6_K: part g the
//        low bytes of 16-value group g, part 4 + g its high bytes),
//        xb [m][XR][chunk] block data: row 0 (s_0, s_1, sx_0, sx_1), row 1
//        (sx_2, sx_3, idx_0, idx_1), row 2 + b block b's four slot values
//        (0 where unused); sx = s * sum x over the block (Q4_K) or the
//        16-value group (Q6_K); idx_b the slots' indices within block b,
//        five bits each (slot j at bits 5j); s_b carries its sign bit set
//        when block b has values taken out.
// F16 weights: fp16 activations as [m][part][chunk] 16-byte units of natural
// pairs, or fp32 activations as [m][part][chunk] units of four floats.
// Columns at or beyond K read as zero; lanes on consecutive chunks read
// consecutive LDS addresses.
#pragma once

#include "chunk.h"

namespace rq {

constexpr float kXMax = 30583.f;  // 7 * (1 + 16 + 256 + 4096): four balanced hex digits
constexpr float kOutlierRatio = 16.f;  // a value at or above amax / kOutlierRatio is large
constexpr int kOutlierSlots = 4;      // values of a block that can be taken out and multiplied exactly

// Work item u = ((m * nch + c) * BLK + b) * 4 + q stages the eight values
// 8q..8q+7 of block b of chunk c of row m. The four items of a block sit in an
// aligned lane quad, which shares the block's maximum and sums through DPP.
template <int FMT>
__device__ __forceinline__ int stage_items(int nch, int M) {
    return M * nch * Traits<FMT>::BLK * 4;
}

// Item u's row m, chunk c, block b and quarter q. At one activation row (M a
// constant 1 after inlining) no division by the chunk count is needed.
struct StagePos {
    int m, c, b, q;
};
template <int FMT>
__device__ __forceinline__ StagePos stage_pos(int u, int nch, int M) {
    constexpr int BLK = Traits<FMT>::BLK;
    const int cb = u >> 2, mc = cb / BLK;
    const int m = M == 1 ? 0 : mc / nch;
    return StagePos{m, mc - m * nch, cb % BLK, u & 3};
}

inline int stage_items_host(int fmt, int64_t nch, int M) {
    return (int)(M * nch * (fmt == Q8_0 ? 1 : 2) * 4);
}

template <bool XF32, bool NORM = false>
struct StageItem {
    uint4 raw[XF32 ? 2 : 1];
    uint4 nw[NORM ? 2 : 1];  // the item's eight norm scales (NORM only)
    uint4 dl[NORM ? 2 : 1];  // the item's eight residual deltas (NORM only)
};

// The rmsnorm prologue's operands (NORM staging, fp32 activations): per-column
// scales, an optional delta added to x first, and where workgroup 0 writes
// x + delta (null elsewhere).
struct NormIn {
    const float* w;
    const float* delta;
    float* x_out;
};

template <int FMT, bool XF32, bool NORM = false>
__device__ __forceinline__ void stage_issue(int u, int nch, int M, int K, const void* xv, int64_t ldx,
                                            StageItem<XF32, NORM>& it, const NormIn& nin = NormIn{}) {
    constexpr int CW = Traits<FMT>::CW;
    const auto [m, c, b, q] = stage_pos<FMT>(u, nch, M);
    int k0 = c * CW + b * 32 + q * 8;
    k0 = k0 < K ? k0 : K - 8;
    if constexpr (XF32) {
        const float* xm = static_cast<const float*>(xv) + (int64_t)m * ldx + k0;
        it.raw[0] = *reinterpret_cast<const uint4*>(xm);
        it.raw[1] = *reinterpret_cast<const uint4*>(xm + 4);
        if constexpr (NORM) {
            it.nw[0] = *reinterpret_cast<const uint4*>(nin.w + k0);
            it.nw[1] = *reinterpret_cast<const uint4*>(nin.w + k0 + 4);
            if (nin.delta) {
                it.dl[0] = *reinterpret_cast<const uint4*>(nin.delta + k0);
                it.dl[1] = *reinterpret_cast<const uint4*>(nin.delta + k0 + 4);
            } else {
                it.dl[0] = it.dl[1] = make_uint4(0, 0, 0, 0);
            }
        }
    } else {
        it.raw[0] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(xv) + (int64_t)m * ldx + k0);
    }
}

typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));

template <int CTRL>
__device__ __forceinline__ int dpp_i32(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_quad_f32(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}

// The four signed-nibble digit words of eight values from their 16-bit
// patterns offset by 0x8888: P[j] holds (x_2j + 0x8888) in its low half and
// (x_2j+1 + 0x8888) in its high half, so every byte of P is a pair of digits
// d_i + 8 and each byte XOR 0x88 a pair of signed digits. Word i of the
// result holds digit i of x_0..x_7 in nibbles 0..7.
__device__ __forceinline__ void digit_words(const uint32_t (&P)[4], uint32_t (&out)[4]) {
    // bytes of x_1, x_0, x_3, x_2 (and x_5, x_4, x_7, x_6): low bytes (digits
    // 0, 1) in A, B; high bytes (digits 2, 3) in C, D
    const uint32_t A = __builtin_amdgcn_perm(P[1], P[0], 0x04060002u), C = __builtin_amdgcn_perm(P[1], P[0], 0x05070103u);
    const uint32_t B = __builtin_amdgcn_perm(P[3], P[2], 0x04060002u), D = __builtin_amdgcn_perm(P[3], P[2], 0x05070103u);
    // Z's low nibbles (signed: ^ 8) z_1, z_0, z_3, z_2 per byte; z | z << 12
    // puts z_0 | z_1 << 4 in byte 1 and z_2 | z_3 << 4 in byte 3
    auto lo = [](uint32_t Z) {
        const uint32_t z = (Z & 0x0F0F0F0Fu) ^ 0x08080808u;
        return z | (z << 12);
    };
    auto hi = [](uint32_t Z) {
        const uint32_t z = ((Z >> 4) & 0x0F0F0F0Fu) ^ 0x08080808u;
        return z | (z << 12);
    };
    out[0] = __builtin_amdgcn_perm(lo(B), lo(A), 0x07050301u);
    out[1] = __builtin_amdgcn_perm(hi(B), hi(A), 0x07050301u);
    out[2] = __builtin_amdgcn_perm(lo(D), lo(C), 0x07050301u);
    out[3] = __builtin_amdgcn_perm(hi(D), hi(C), 0x07050301u);
}

// Encodes eight values of a 32-value block whose maximum magnitude is amax
// (the values finite, |v| <= amax): x = rint(v / s) with the block scale
// s = amax / 30583, as digit words (nibble formats: four words, one per
// balanced hex digit; Q8_0: two low-byte words, then two high-byte words), the
// integer sum of the eight in `sum`; returns s. 1 / s is the hardware
// reciprocal (within one ulp), so |v / s| stays below 30583.5 and needs no
// clamp. A block whose step would fall below the smallest normal float (amax
// under 30583 * 2^-126) takes the step 2^-126. The rounding is one fma with
// 1.5 * 2^23 + c, c = 0x8888 (nibble formats) or 0x8080 (Q8_0): the sum lies
// in [2^23, 2^24), where a float's pattern is 0x4B000000 plus its value
// minus 2^23, so it is rint(v / s) + c (to nearest even: c is even) in the
// pattern's low bits and the offset digits come out of the low 16 bits as
// they are.
template <int FMT>
__device__ __forceinline__ float encode_item(const float (&v)[8], float amax, uint32_t (&w4)[4], int& sum) {
    constexpr bool kBytes = FMT == Q8_0 || FMT == Q6_K;
    constexpr float kOffset = kBytes ? 32896.f : 34952.f;  // 0x8080, 0x8888
    constexpr float kMagic = 12582912.0f + kOffset;              // 1.5 * 2^23 + c
    constexpr uint32_t kMagicBits = 0x4B400000u + (uint32_t)kOffset;
    float s = amax * (1.0f / kXMax);
    const bool tiny = s < 0x1p-126f;  // (zero or tiny blocks)
    float inv = __builtin_amdgcn_rcpf(s);
    inv = tiny ? (amax > 0.f ? 0x1p126f : 0.f) : inv;
    s = tiny ? (amax > 0.f ? 0x1p-126f : 0.f) : s;
    uint32_t xb[8];
    uint32_t usum = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        xb[k] = __builtin_bit_cast(uint32_t, fmaf(v[k], inv, kMagic));
        usum += xb[k];
    }
    sum = (int)(usum - 8u * kMagicBits);
    uint32_t P[4];  // (x_2j + c) | (x_2j+1 + c) << 16
#pragma unroll
    for (int j = 0; j < 4; ++j) P[j] = __builtin_amdgcn_perm(xb[2 * j + 1], xb[2 * j], 0x05040100u);
    if constexpr (FMT == Q8_0) {
        // low bytes of x_0..x_3 (x_4..x_7), then the high bytes; ^ 0x80 per byte
        w4[0] = __builtin_amdgcn_perm(P[1], P[0], 0x06040200u) ^ 0x80808080u;
        w4[1] = __builtin_amdgcn_perm(P[3], P[2], 0x06040200u) ^ 0x80808080u;
        w4[2] = __builtin_amdgcn_perm(P[1], P[0], 0x07050301u) ^ 0x80808080u;
        w4[3] = __builtin_amdgcn_perm(P[3], P[2], 0x07050301u) ^ 0x80808080u;
    } else if constexpr (FMT == Q6_K) {
        // low bytes of x_0, x_2, x_4, x_6 and of x_1, x_3, x_5, x_7, then their
        // high bytes (the order of the weights' byte words, chunk.h)
        const uint32_t e0 = __builtin_amdgcn_perm(xb[2], xb[0], 0x05010400u);  // lo 0, lo 2, hi 0, hi 2
        const uint32_t e1 = __builtin_amdgcn_perm(xb[6], xb[4], 0x05010400u);
        const uint32_t o0 = __builtin_amdgcn_perm(xb[3], xb[1], 0x05010400u);
        const uint32_t o1 = __builtin_amdgcn_perm(xb[7], xb[5], 0x05010400u);
        w4[0] = __builtin_amdgcn_perm(e1, e0, 0x05040100u) ^ 0x80808080u;
        w4[1] = __builtin_amdgcn_perm(o1, o0, 0x05040100u) ^ 0x80808080u;
        w4[2] = __builtin_amdgcn_perm(e1, e0, 0x07060302u) ^ 0x80808080u;
        w4[3] = __builtin_amdgcn_perm(o1, o0, 0x07060302u) ^ 0x80808080u;
    } else {
        digit_words(P, w4);
    }
    return s;
}

// Encodes item u and stores it into LDS. Every lane of the item's quad must
// run it together (the block maximum and sums move through DPP).
// Returns whether the item's block has values taken out.
template <int FMT, bool XF32, bool NORM = false>
__device__ __forceinline__ bool stage_finish(int u, int nch, int M, int K, const StageItem<XF32, NORM>& it,
                                             uint4* xd, float* xbf, const NormIn& nin = NormIn{},
                                             float* ss = nullptr) {
    constexpr int CW = Traits<FMT>::CW, BLK = Traits<FMT>::BLK, XP = Traits<FMT>::XP, XR = Traits<FMT>::XR;
    const auto [m, c, b, q] = stage_pos<FMT>(u, nch, M);
    const bool live = c * CW + b * 32 < K;
    float v[8];
    if constexpr (XF32) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            v[t] = __builtin_bit_cast(float, word(it.raw[0], t));
            v[4 + t] = __builtin_bit_cast(float, word(it.raw[1], t));
        }
        if constexpr (NORM) {
            // u = x + delta; its squares for the norm and (workgroup 0) its
            // copy; then rmsnorm's per-column scale (the common factor is
            // applied to the products)
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                v[t] += __builtin_bit_cast(float, word(it.dl[0], t));
                v[4 + t] += __builtin_bit_cast(float, word(it.dl[1], t));
            }
            if (c * CW + b * 32 < K) {
                float s2 = 0.f;
#pragma unroll
                for (int k = 0; k < 8; ++k) s2 = fmaf(v[k], v[k], s2);
                *ss += s2;
                if (nin.x_out) {
                    float* xo = nin.x_out + (c * CW + b * 32 + q * 8);
                    *reinterpret_cast<float4*>(xo) = make_float4(v[0], v[1], v[2], v[3]);
                    *reinterpret_cast<float4*>(xo + 4) = make_float4(v[4], v[5], v[6], v[7]);
                }
            }
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                v[t] *= __builtin_bit_cast(float, word(it.nw[0], t));
                v[4 + t] *= __builtin_bit_cast(float, word(it.nw[1], t));
            }
        }
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[2 * e] = half_lo(word(it.raw[0], e));
            v[2 * e + 1] = half_hi(word(it.raw[0], e));
        }
    }
    // A NaN or an infinity anywhere in the block makes the block's scale NaN
    // (its digits are zero), so every product that reads the block is NaN:
    // a non-finite activation is never dropped by the maximum or the rounding.
    // Magnitudes compared as bit patterns (sign cleared): for finite values
    // their integer order is their order, and every infinity or NaN pattern
    // lies above the largest finite one, so one maximum finds both the
    // block's largest magnitude and whether any value is not finite.
    uint32_t i1 = 0, i2 = 0;  // this item's largest and second largest magnitudes, as fp32 patterns
    if constexpr (XF32) {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t mk = __builtin_bit_cast(uint32_t, v[k]) & 0x7FFFFFFFu;
            i2 = max(i2, min(i1, mk));
            i1 = max(i1, mk);
        }
    } else {
        // fp16 patterns order the same way, two to a word (packed 16-bit
        // maxima); the two largest then convert exactly to fp32
        u16x2_t hi, lo;
        {
            const u16x2_t m0 = __builtin_bit_cast(u16x2_t, word(it.raw[0], 0) & 0x7FFF7FFFu);
            const u16x2_t m1 = __builtin_bit_cast(u16x2_t, word(it.raw[0], 1) & 0x7FFF7FFFu);
            const u16x2_t m2 = __builtin_bit_cast(u16x2_t, word(it.raw[0], 2) & 0x7FFF7FFFu);
            const u16x2_t m3 = __builtin_bit_cast(u16x2_t, word(it.raw[0], 3) & 0x7FFF7FFFu);
            hi = __builtin_elementwise_max(m0, m1);
            lo = __builtin_elementwise_min(m0, m1);
            lo = __builtin_elementwise_max(lo, __builtin_elementwise_min(hi, m2));
            hi = __builtin_elementwise_max(hi, m2);
            lo = __builtin_elementwise_max(lo, __builtin_elementwise_min(hi, m3));
            hi = __builtin_elementwise_max(hi, m3);
        }
        const uint32_t h1 = max((uint32_t)hi.x, (uint32_t)hi.y);
        const uint32_t h2 = max(min((uint32_t)hi.x, (uint32_t)hi.y), max((uint32_t)lo.x, (uint32_t)lo.y));
        i1 = __builtin_bit_cast(uint32_t, half_lo(h1));
        i2 = __builtin_bit_cast(uint32_t, half_lo(h2));
    }
    uint32_t bbits = i1;
    bbits = max(bbits, (uint32_t)dpp_i32<0xB1>((int)bbits));  // quad_perm [1,0,3,2]
    bbits = max(bbits, (uint32_t)dpp_i32<0x4E>((int)bbits));  // quad_perm [2,3,0,1]
    const int bad = bbits > 0x7F7FFFFFu;
    float amax = __builtin_bit_cast(float, bbits);
    if (!live) amax = 0.f;
    // Values are taken out only when at most kOutlierSlots of the block are
    // at or above amax / kOutlierRatio. Each item's two largest count at most
    // the large values; when they already exceed kOutlierSlots (ordinary
    // activations, always) nothing is taken out. Otherwise the values are
    // counted and taken out in rounds (a rare, quad-uniform branch).
    const uint32_t thr0 = __builtin_bit_cast(uint32_t, amax * (1.0f / kOutlierRatio));
    int seen = (int)(i1 >= thr0) + (int)(i2 >= thr0);
    seen += dpp_i32<0xB1>(seen);
    seen += dpp_i32<0x4E>(seen);
    bool outlier = false;
    float slot[4] = {0.f, 0.f, 0.f, 0.f};  // the block's slot values (each set by its owner's lane)
    uint32_t sidx = 0;                      // their indices in the block, five bits per slot
    if (__builtin_expect(seen <= kOutlierSlots && live && !bad, 0)) {
        uint32_t mb[8];  // the magnitudes, as fp32 patterns
#pragma unroll
        for (int k = 0; k < 8; ++k) mb[k] = __builtin_bit_cast(uint32_t, v[k]) & 0x7FFFFFFFu;
        uint32_t cur = bbits;  // the largest magnitude not taken out
        int used = 0;
        uint32_t taken = 0;  // bit k: v[k] is taken out
        for (int round = 0; round < kOutlierSlots && cur != 0; ++round) {
            const uint32_t thr = __builtin_bit_cast(uint32_t, __builtin_bit_cast(float, cur) * (1.0f / kOutlierRatio));
            int n = 0;
#pragma unroll
            for (int k = 0; k < 8; ++k) n += !((taken >> k) & 1u) && mb[k] >= thr;
            int tot = n + dpp_i32<0xB1>(n);
            tot += dpp_i32<0x4E>(tot);
            if (tot > kOutlierSlots - used) break;
            // this lane's first slot: the slots used so far plus the lower lanes' counts
            const int n0 = dpp_i32<0x00>(n), n1 = dpp_i32<0x55>(n), n2 = dpp_i32<0xAA>(n);
            int pos = used + (q > 0 ? n0 : 0) + (q > 1 ? n1 : 0) + (q > 2 ? n2 : 0);
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                if (!((taken >> k) & 1u) && mb[k] >= thr) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) slot[j] = pos == j ? v[k] : slot[j];
                    sidx |= (uint32_t)(q * 8 + k) << (5 * pos);
                    taken |= 1u << k;
                    ++pos;
                }
            }
            used += tot;
            uint32_t rest = 0;
#pragma unroll
            for (int k = 0; k < 8; ++k) rest = ((taken >> k) & 1u) ? rest : max(rest, mb[k]);
            rest = max(rest, (uint32_t)dpp_i32<0xB1>((int)rest));
            rest = max(rest, (uint32_t)dpp_i32<0x4E>((int)rest));
            cur = rest;
        }
        if (used > 0) {  // (quad-uniform) the block is scaled by what is left
            outlier = true;
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] = ((taken >> k) & 1u) ? 0.f : v[k];
            amax = __builtin_bit_cast(float, cur);
            // every slot has one owner and zeros elsewhere: the quad's sum is its value
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                slot[j] += dpp_quad_f32<0xB1>(slot[j]);
                slot[j] += dpp_quad_f32<0x4E>(slot[j]);
            }
            sidx += (uint32_t)dpp_i32<0xB1>((int)sidx);
            sidx += (uint32_t)dpp_i32<0x4E>((int)sidx);
        }
    }
    if (__builtin_expect(bad, 0)) {
        amax = 0.f;
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = 0.f;
    }
    uint32_t w4[4];
    int sum;
    float s = encode_item<FMT>(v, amax, w4, sum);
    if (bad && live) s = __builtin_nanf("");
    uint32_t* xdw = reinterpret_cast<uint32_t*>(xd);
    if constexpr (FMT == Q8_0) {
        // low-byte words 2q, 2q+1 in parts 0-1, high-byte words in parts 2-3
        const int part = q >> 1, comp = (q & 1) * 2;
        uint32_t* lo_at = xdw + ((m * XP + part) * nch + c) * 4 + comp;
        uint32_t* hi_at = xdw + ((m * XP + 2 + part) * nch + c) * 4 + comp;
        lo_at[0] = w4[0];
        lo_at[1] = w4[1];
        hi_at[0] = w4[2];
        hi_at[1] = w4[3];
    } else if constexpr (FMT == Q6_K) {
        // group g = 2b + q/2: low-byte words in part g, high-byte words in
        // part 4 + g; values 0-7 of the group in components 0-1, 8-15 in 2-3
        const int g = 2 * b + (q >> 1), comp = (q & 1) * 2;
        uint32_t* lo_at = xdw + ((m * XP + g) * nch + c) * 4 + comp;
        uint32_t* hi_at = xdw + ((m * XP + 4 + g) * nch + c) * 4 + comp;
        lo_at[0] = w4[0];
        lo_at[1] = w4[1];
        hi_at[0] = w4[2];
        hi_at[1] = w4[3];
    } else {
        // digit i, word 4b + q of the chunk: part 2i + b, component q
#pragma unroll
        for (int i = 0; i < 4; ++i) xdw[((m * XP + 2 * i + b) * nch + c) * 4 + q] = w4[i];
    }
    // block data rows 0 (s_0, s_1, sx_0, sx_1) and 1 (sx_2, sx_3, idx_0, idx_1), slot row 2 + b
    const int pair = sum + dpp_i32<0xB1>(sum);   // this half block (16 values)
    const int whole = pair + dpp_i32<0x4E>(pair);  // the block
    float* b0 = xbf + ((m * XR + 0) * nch + c) * 4;
    float* b1 = xbf + ((m * XR + 1) * nch + c) * 4;
    if (q == 0) {
        b0[b] = outlier ? -s : s;  // the sign bit marks a block with values taken out (s >= 0 otherwise)
        reinterpret_cast<uint32_t*>(b1)[2 + b] = sidx;
        *reinterpret_cast<float4*>(xbf + ((m * XR + 2 + b) * nch + c) * 4) =
            make_float4(slot[0], slot[1], slot[2], slot[3]);
        if constexpr (BLK == 1) {
            b0[1] = 0.f;  // (read with s_0 for the outlier mark)
            reinterpret_cast<uint32_t*>(b1)[3] = 0u;
        }
    }
    if constexpr (FMT == Q4_K) {
        if (q == 0) b0[2 + b] = s * (float)whole;
    } else if constexpr (FMT == Q6_K) {
        if ((q & 1) == 0) {  // groups 2b (q = 0) and 2b + 1 (q = 2)
            const int g = 2 * b + (q >> 1);
            const float sx = s * (float)pair;
            if (g < 2) b0[2 + g] = sx; else b1[g - 2] = sx;
        }
    }
    return outlier;
}

// A workgroup-uniform "some staged block holds an outlier", from each
// thread's own answer: one word per wave in `wave_flags` (every wave writes
// its own), read back after the barrier that follows the staging.
__device__ __forceinline__ void publish_outliers(bool mine, int* wave_flags) {
    const bool any = __builtin_amdgcn_ballot_w64(mine) != 0;
    if ((threadIdx.x & 63) == 0) wave_flags[threadIdx.x >> 6] = any ? 1 : 0;
}
__device__ __forceinline__ bool read_outliers(const int* wave_flags, int nthreads) {
    int any = 0;
    for (int i = 0; i < (nthreads >> 6); ++i) any |= wave_flags[i];
    return __builtin_amdgcn_readfirstlane(any) != 0;
}

// Staging with up to NJ items per thread: all activation loads are issued
// before the caller's weight loads (stage_multi_issue), encoded afterwards
// (stage_multi_finish). kStageNJ by default; the norm prologue's items carry
// three times the registers, and the two-waves-per-tile kernel (at most 128
// registers a lane) takes kStageNJNorm of them.
constexpr int kStageNJ = 4;
constexpr int kStageNJNorm = 2;

// `nthreads` is the workgroup's size, passed in rather than read from the
// dispatch packet (blockDim), whose read is a memory round trip at the start
// of every workgroup.
template <int FMT, bool XF32, bool NORM = false, int NJ = kStageNJ>
__device__ __forceinline__ void stage_multi_issue(int nch, int K, const void* x, int64_t ldx, int M, int nthreads,
                                                  StageItem<XF32, NORM> (&it)[NJ],
                                                  const NormIn& nin = NormIn{}) {
    const int total = stage_items<FMT>(nch, M);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        // (rounds past the last item are skipped by the whole workgroup; a
        // thread past it in the last round loads an item of its own quad)
        if (j * nthreads >= total) break;
        const int u = (int)threadIdx.x + j * nthreads;
        stage_issue<FMT, XF32, NORM>(u < total ? u : (int)threadIdx.x % 4, nch, M, K, x, ldx, it[j], nin);
    }
}

template <int FMT, bool XF32, bool NORM = false, int NJ = kStageNJ>
__device__ __forceinline__ bool stage_multi_finish(int nch, int K, int M, int nthreads,
                                                   const StageItem<XF32, NORM> (&it)[NJ], uint4* xd, float* xbf,
                                                   const NormIn& nin = NormIn{}, float* ss = nullptr) {
    const int total = stage_items<FMT>(nch, M);
    bool out = false;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        if (j * nthreads >= total) break;
        const int u = (int)threadIdx.x + j * nthreads;
        if (u < total) out |= stage_finish<FMT, XF32, NORM>(u, nch, M, K, it[j], xd, xbf, nin, ss);
    }
    return out;
}

// Plain loop (used when a block has more items than kStageNJ per thread).
template <int FMT, bool XF32, bool NORM = false>
__device__ __forceinline__ bool stage_all(int nch, int K, const void* x, int64_t ldx, int M, int nthreads, uint4* xd,
                                          float* xbf, const NormIn& nin = NormIn{}, float* ss = nullptr) {
    const int total = stage_items<FMT>(nch, M);
    bool out = false;
    for (int u = threadIdx.x; u < total; u += nthreads) {
        StageItem<XF32, NORM> it;
        stage_issue<FMT, XF32, NORM>(u, nch, M, K, x, ldx, it, nin);
        out |= stage_finish<FMT, XF32, NORM>(u, nch, M, K, it, xd, xbf, nin, ss);
    }
    return out;
}

// LDS bytes of a staged activation block for the integer kernels: digit
// words, then xb [m][XR][chunk] (block data and the slot rows).
__host__ __device__ inline size_t stage_bytes_int(int fmt, int M, int nch) {
    const int xp = fmt == Q8_0 ? 4 : 8, xr = fmt == Q8_0 ? 3 : 4;
    return (size_t)M * nch * (size_t)(xp + xr) * 16;
}

// F16 weights: fp16 activations as natural pairs, or fp32 activations. Up to
// kCopyNJ units per thread are all loaded before any is stored, so the copy
// costs one round trip; larger rows loop.
constexpr int kCopyNJ = 4;

__device__ __forceinline__ void stage_f16_pairs(int nch, int K, const void* xv, int64_t ldx, int M, int nthreads,
                                                uint4* xq) {
    const uint16_t* x = static_cast<const uint16_t*>(xv);
    const int total = M * 8 * nch;
    auto unit = [&](int u) {
        const int c = u % nch, mj = u / nch, j = mj % 8, m = mj / 8;
        const int k0 = c * 64 + j * 8;
        return k0 < K ? *reinterpret_cast<const uint4*>(x + (int64_t)m * ldx + k0) : make_uint4(0, 0, 0, 0);
    };
    if (total <= kCopyNJ * nthreads) {
        uint4 v[kCopyNJ];
#pragma unroll
        for (int j = 0; j < kCopyNJ; ++j) {
            const int u = (int)threadIdx.x + j * nthreads;
            if (u < total) v[j] = unit(u);
        }
#pragma unroll
        for (int j = 0; j < kCopyNJ; ++j) {
            const int u = (int)threadIdx.x + j * nthreads;
            if (u < total) xq[u] = v[j];
        }
        return;
    }
    for (int u = threadIdx.x; u < total; u += nthreads) xq[u] = unit(u);
}

__device__ __forceinline__ void stage_f32_quads(int nch, int K, const void* xv, int64_t ldx, int M, int nthreads,
                                                float4* xf) {
    const float* x = static_cast<const float*>(xv);
    const int total = M * 16 * nch;
    auto unit = [&](int u) {
        const int c = u % nch, mj = u / nch, j = mj % 16, m = mj / 16;
        const int k0 = c * 64 + j * 4;
        return k0 < K ? *reinterpret_cast<const float4*>(x + (int64_t)m * ldx + k0) : make_float4(0.f, 0.f, 0.f, 0.f);
    };
    if (total <= kCopyNJ * nthreads) {
        float4 v[kCopyNJ];
#pragma unroll
        for (int j = 0; j < kCopyNJ; ++j) {
            const int u = (int)threadIdx.x + j * nthreads;
            if (u < total) v[j] = unit(u);
        }
#pragma unroll
        for (int j = 0; j < kCopyNJ; ++j) {
            const int u = (int)threadIdx.x + j * nthreads;
            if (u < total) xf[u] = v[j];
        }
        return;
    }
    for (int u = threadIdx.x; u < total; u += nthreads) xf[u] = unit(u);
}

__host__ __device__ inline size_t stage_bytes_f16w(int xtype_f32, int M, int nch) {
    return (size_t)M * nch * (xtype_f32 ? 16 : 8) * 16;
}

// DPP lane moves (VALU modifiers, no LDS traffic). Lanes outside row_mask
// read 0.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_f32(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xf, false));
}

// Sum over the G lanes of each aligned lane group (G = 8, 16, 32 or 64); the
// total lands in the group's last lane (g == G - 1; for G <= 16 in every lane).
// quad_perm [1,0,3,2] and [2,3,0,1], row_half_mirror, row_mirror, then
// row_bcast:15 (rows 1, 3) and row_bcast:31 (rows 2, 3).
__device__ __forceinline__ float group_sum(float v, int G) {
    v += dpp_f32<0xB1, 0xf>(v);
    v += dpp_f32<0x4E, 0xf>(v);
    v += dpp_f32<0x141, 0xf>(v);
    if (G >= 16) v += dpp_f32<0x140, 0xf>(v);
    if (G >= 32) v += dpp_f32<0x142, 0xa>(v);
    if (G >= 64) v += dpp_f32<0x143, 0xc>(v);
    return v;
}

// Dot of one F16-weight chunk against staged fp32 activations (exact products).
__device__ __forceinline__ float chunk_dot_f32(const ChunkData<F16>& d, const float4* xf, int nch, int c, int m) {
    float w[64];
    decode_chunk<F16>(d, c, w);
    float a = 0.f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const float4 xv = xf[(m * 16 + j) * nch + c];
        a = fmaf(w[4 * j], xv.x, a);
        a = fmaf(w[4 * j + 1], xv.y, a);
        a = fmaf(w[4 * j + 2], xv.z, a);
        a = fmaf(w[4 * j + 3], xv.w, a);
    }
    return a;
}

}  // namespace rq
