// Host-side loader repack: GGUF block bytes <-> the kernel's HBM layout
// (layout.h). Both directions are exact bijections on the bits (plus Q4_0's
// odd-row padding and 16-byte row alignment), so unpack(repack(b)) == b.
//
// Reference counterpart: recipe's batch-1 loader interleaves rows four bytes at
// a time across the lanes of a wave (recipe.rs:3162-3212 row_interleave /
// interleave_rows, applied by Buffer::fill_weights at recipe.rs:26980-27010).
// This layout instead gives each lane whole 16-byte parts of one row, makes
// every load instruction of a wave one contiguous 1 KiB run, and keeps each
// group's scales beside its codes.
#include "repack.h"

#include <string.h>

namespace rq {

static inline uint8_t q6_code(const uint8_t* blk, int i) {
    // Field positions of dequant_q6k (recipe.rs:3743-3780).
    int chunk = i / 128, local = i % 128, group = local / 32, within = local % 32;
    int lo = (blk[chunk * 64 + within + 32 * (group & 1)] >> (4 * (group / 2))) & 15;
    int hi = (blk[128 + chunk * 32 + within] >> (2 * group)) & 3;
    return (uint8_t)(lo | (hi << 4));
}

static inline void q6_store(uint8_t* blk, int i, int q) {
    int chunk = i / 128, local = i % 128, group = local / 32, within = local % 32;
    uint8_t& lo = blk[chunk * 64 + within + 32 * (group & 1)];
    int sh = 4 * (group / 2);
    lo = (uint8_t)((lo & ~(15 << sh)) | ((q & 15) << sh));
    uint8_t& hi = blk[128 + chunk * 32 + within];
    int hs = 2 * group;
    hi = (uint8_t)((hi & ~(3 << hs)) | (((q >> 4) & 3) << hs));
}

// 32 four-bit codes in natural order, XOR 8, two per byte (layout.h).
static void pack_nibbles(const uint8_t* q, uint8_t* out16) {
    for (int j = 0; j < 16; ++j) out16[j] = (uint8_t)(((q[2 * j] ^ 8) & 15) | (((q[2 * j + 1] ^ 8) & 15) << 4));
}

static void unpack_nibbles(const uint8_t* in16, uint8_t* q) {
    for (int j = 0; j < 16; ++j) {
        q[2 * j] = (uint8_t)((in16[j] & 15) ^ 8);
        q[2 * j + 1] = (uint8_t)((in16[j] >> 4) ^ 8);
    }
}

// Q6_K high fields of one 16-weight group as one word (layout.h).
static uint32_t q6_high_word(const uint8_t* q6) {
    uint32_t w = 0;
    for (int j = 0; j < 8; ++j) {
        w |= (uint32_t)((q6[j] >> 4) & 3) << (4 * j);
        w |= (uint32_t)((q6[8 + j] >> 4) & 3) << (4 * j + 2);
    }
    return w;
}

// Q4_K scales: the 12 k_scale bytes of a superblock (bytes 4..15 of the
// block; get_scale_min_k4, recipe.rs:15204-15210: sub-block j < 4 has scale
// s[j] & 63 and minimum s[j + 4] & 63, j >= 4 has scale (s[j + 4] & 15) |
// (s[j - 4] >> 6) << 4 and minimum (s[j + 4] >> 4) | (s[j] >> 6) << 4) <->
// the layout's four 24-bit fields, one per chunk p (sub-blocks 2p, 2p + 1):
// bits 24p.. of the 96-bit little-endian value hold scale(2p), min(2p),
// scale(2p + 1), min(2p + 1), six bits each. Both hold the same 96 bits.
static void q4k_fields_from_kscale(const uint8_t* s, uint8_t* out12) {
    uint8_t sc[8], mn[8];
    for (int j = 0; j < 4; ++j) {
        sc[j] = s[j] & 63;
        mn[j] = s[j + 4] & 63;
        sc[j + 4] = (uint8_t)((s[j + 8] & 15) | ((s[j] >> 6) << 4));
        mn[j + 4] = (uint8_t)((s[j + 8] >> 4) | ((s[j + 4] >> 6) << 4));
    }
    uint64_t lo = 0, hi = 0;  // the 96 bits: lo = bits 0..63, hi = bits 64..95
    for (int p = 0; p < 4; ++p) {
        const uint64_t f = (uint64_t)sc[2 * p] | (uint64_t)mn[2 * p] << 6 | (uint64_t)sc[2 * p + 1] << 12 |
                           (uint64_t)mn[2 * p + 1] << 18;
        const int at = 24 * p;
        if (at + 24 <= 64) lo |= f << at;
        else if (at >= 64) hi |= f << (at - 64);
        else {
            lo |= f << at;
            hi |= f >> (64 - at);
        }
    }
    for (int i = 0; i < 8; ++i) out12[i] = (uint8_t)(lo >> (8 * i));
    for (int i = 0; i < 4; ++i) out12[8 + i] = (uint8_t)(hi >> (8 * i));
}

static void q4k_kscale_from_fields(const uint8_t* in12, uint8_t* s) {
    uint64_t lo = 0, hi = 0;
    for (int i = 0; i < 8; ++i) lo |= (uint64_t)in12[i] << (8 * i);
    for (int i = 0; i < 4; ++i) hi |= (uint64_t)in12[8 + i] << (8 * i);
    uint8_t sc[8], mn[8];
    for (int p = 0; p < 4; ++p) {
        const int at = 24 * p;
        uint64_t f;
        if (at + 24 <= 64) f = lo >> at;
        else if (at >= 64) f = hi >> (at - 64);
        else f = (lo >> at) | (hi << (64 - at));
        sc[2 * p] = f & 63;
        mn[2 * p] = (f >> 6) & 63;
        sc[2 * p + 1] = (f >> 12) & 63;
        mn[2 * p + 1] = (f >> 18) & 63;
    }
    for (int j = 0; j < 4; ++j) {
        s[j] = (uint8_t)(sc[j] | ((sc[j + 4] >> 4) << 6));
        s[j + 4] = (uint8_t)(mn[j] | ((mn[j + 4] >> 4) << 6));
        s[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4));
    }
}

// Shapes the kernels take: rows below 2^31 (their row indices are 32-bit)
// and cols at most 2^30, a whole number of blocks; both products below are
// then checked for overflow, so that a shape read from an untrusted file
// cannot wrap a size.
static bool shape_ok(int fmt, int64_t rows, int64_t cols) {
    FormatInfo f = format_info(fmt);
    if (f.block_values == 0 || rows <= 0 || cols <= 0) return false;
    if (rows > kMaxRows || cols > kMaxCols) return false;
    if (cols % f.block_values != 0) return false;
    if (cols % 32 != 0) return false;
    if (fmt == F16 && cols % 64 != 0) return false;
    return true;
}

int64_t gguf_bytes(int fmt, int64_t rows, int64_t cols) {
    FormatInfo f = format_info(fmt);
    if (!shape_ok(fmt, rows, cols)) return -1;
    int64_t n;
    if (__builtin_mul_overflow(rows, (cols / f.block_values) * f.block_bytes, &n)) return -1;
    return n;
}

int64_t layout_bytes(int fmt, int64_t rows, int64_t cols) {
    if (!shape_ok(fmt, rows, cols)) return -1;
    int64_t n;
    if (__builtin_mul_overflow(rows, row_bytes(fmt, cols), &n)) return -1;
    return n;
}

// Copies one chunk between its GGUF blocks (a row's block bytes) and the
// layout (a row's repacked bytes): TO_LAYOUT reads `blocks` and writes `row`,
// otherwise it reads `row` and writes `blocks`.
template <bool TO_LAYOUT>
static void chunk_copy(int fmt, const uint8_t* src_blocks, uint8_t* dst_blocks, const uint8_t* src_row, uint8_t* dst_row,
                       int64_t c, int64_t nch, int64_t nblk) {
    const ChunkPlace pl = chunk_place(fmt, c, nch);
    const int64_t meta = meta_offset(fmt, c, nch);
    auto part = [&](int p) { return code_offset(fmt, c, p, nch); };
    switch (fmt) {
        case Q8_0: {
            if (TO_LAYOUT) {
                const uint8_t* blk = src_blocks + c * 34;
                memcpy(dst_row + meta + 2 * pl.within, blk, 2);
                for (int p = 0; p < 2; ++p) memcpy(dst_row + part(p), blk + 2 + 16 * p, 16);
            } else {
                uint8_t* blk = dst_blocks + c * 34;
                memcpy(blk, src_row + meta + 2 * pl.within, 2);
                for (int p = 0; p < 2; ++p) memcpy(blk + 2 + 16 * p, src_row + part(p), 16);
            }
            break;
        }
        case Q4_0: {
            for (int p = 0; p < 2; ++p) {
                const int64_t b = 2 * c + p;
                const int64_t d_at = meta + 4 * pl.within + 2 * p;
                if (TO_LAYOUT) {
                    if (b < nblk) {
                        const uint8_t* blk = src_blocks + b * 18;
                        memcpy(dst_row + d_at, blk, 2);
                        uint8_t q[32];
                        for (int i = 0; i < 16; ++i) {
                            q[i] = blk[2 + i] & 15;  // byte i: weight i low nibble, i + 16 high
                            q[i + 16] = blk[2 + i] >> 4;
                        }
                        pack_nibbles(q, dst_row + part(p));
                    } else {
                        memset(dst_row + d_at, 0, 2);
                        memset(dst_row + part(p), 0, 16);  // q = 8: (q - 8) * d = 0
                    }
                } else if (b < nblk) {
                    uint8_t* blk = dst_blocks + b * 18;
                    memcpy(blk, src_row + d_at, 2);
                    uint8_t q[32];
                    unpack_nibbles(src_row + part(p), q);
                    for (int i = 0; i < 16; ++i) blk[2 + i] = (uint8_t)((q[i] & 15) | ((q[i + 16] & 15) << 4));
                }
            }
            break;
        }
        case Q4_K: {
            const int64_t sb = c / 4;
            const int p = (int)(c % 4);
            const int64_t m_at = meta + (pl.within / 4) * 16;
            if (TO_LAYOUT) {
                const uint8_t* blk = src_blocks + sb * 144;
                if (p == 0) {
                    memcpy(dst_row + m_at, blk, 4);  // d, dmin
                    q4k_fields_from_kscale(blk + 4, dst_row + m_at + 4);
                }
                for (int h = 0; h < 2; ++h) {  // sub-block 2p + h: low or high nibbles of bytes 32p..32p+31
                    uint8_t q[32];
                    for (int i = 0; i < 32; ++i) q[i] = (blk[16 + 32 * p + i] >> (4 * h)) & 15;
                    pack_nibbles(q, dst_row + part(h));
                }
            } else {
                uint8_t* blk = dst_blocks + sb * 144;
                if (p == 0) {
                    memcpy(blk, src_row + m_at, 4);
                    q4k_kscale_from_fields(src_row + m_at + 4, blk + 4);
                }
                uint8_t lo[32], hi[32];
                unpack_nibbles(src_row + part(0), lo);
                unpack_nibbles(src_row + part(1), hi);
                for (int i = 0; i < 32; ++i) blk[16 + 32 * p + i] = (uint8_t)(lo[i] | (hi[i] << 4));
            }
            break;
        }
        case Q6_K: {
            const int64_t sb = c / 4;
            const int t = (int)(c % 4);
            const int64_t sc_at = meta + (pl.within / 4) * 16;
            const int64_t d_at = meta + (pl.nb / 4) * 16 + (pl.within / 4) * 2;
            if (TO_LAYOUT) {
                const uint8_t* blk = src_blocks + sb * 210;
                if (t == 0) {
                    memcpy(dst_row + sc_at, blk + 192, 16);
                    memcpy(dst_row + d_at, blk + 208, 2);
                }
                uint8_t q6[64], lo[64];
                for (int e = 0; e < 64; ++e) {
                    q6[e] = q6_code(blk, 64 * t + e);
                    lo[e] = q6[e] & 15;
                }
                pack_nibbles(lo, dst_row + part(0));
                pack_nibbles(lo + 32, dst_row + part(1));
                uint32_t hi[4];
                for (int g = 0; g < 4; ++g) hi[g] = q6_high_word(q6 + 16 * g);
                memcpy(dst_row + part(2), hi, 16);
            } else {
                uint8_t* blk = dst_blocks + sb * 210;
                if (t == 0) {
                    memset(blk, 0, 192);
                    memcpy(blk + 192, src_row + sc_at, 16);
                    memcpy(blk + 208, src_row + d_at, 2);
                }
                uint8_t lo[64];
                unpack_nibbles(src_row + part(0), lo);
                unpack_nibbles(src_row + part(1), lo + 32);
                uint32_t hi[4];
                memcpy(hi, src_row + part(2), 16);
                for (int e = 0; e < 64; ++e) {
                    const int g = e / 16, j = e % 16;
                    const int sh = j < 8 ? 4 * j : 4 * (j - 8) + 2;
                    q6_store(blk, 64 * t + e, lo[e] | (int)(((hi[g] >> sh) & 3) << 4));
                }
            }
            break;
        }
        case F16: {
            for (int p = 0; p < 8; ++p) {
                if (TO_LAYOUT)
                    memcpy(dst_row + part(p), src_blocks + c * 128 + 16 * p, 16);
                else
                    memcpy(dst_blocks + c * 128 + 16 * p, src_row + part(p), 16);
            }
            break;
        }
        default: break;
    }
}

int repack(int fmt, int64_t rows, int64_t cols, const uint8_t* src, uint8_t* dst) {
    if (layout_bytes(fmt, rows, cols) < 0 || gguf_bytes(fmt, rows, cols) < 0) return -1;
    const FormatInfo f = format_info(fmt);
    const int64_t rb = row_bytes(fmt, cols);
    const int64_t nch = chunks_per_row(fmt, cols);
    const int64_t nblk = cols / f.block_values;
    const int64_t src_row = nblk * f.block_bytes;
    memset(dst, 0, (size_t)(rows * rb));
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < nch; ++c)
            chunk_copy<true>(fmt, src + r * src_row, nullptr, nullptr, dst + r * rb, c, nch, nblk);
    return 0;
}

int unpack(int fmt, int64_t rows, int64_t cols, const uint8_t* src, uint8_t* dst) {
    if (layout_bytes(fmt, rows, cols) < 0 || gguf_bytes(fmt, rows, cols) < 0) return -1;
    const FormatInfo f = format_info(fmt);
    const int64_t rb = row_bytes(fmt, cols);
    const int64_t nch = chunks_per_row(fmt, cols);
    const int64_t nblk = cols / f.block_values;
    const int64_t dst_row = nblk * f.block_bytes;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < nch; ++c)
            chunk_copy<false>(fmt, nullptr, dst + r * dst_row, src + r * rb, nullptr, c, nch, nblk);
    return 0;
}

}  // namespace rq
