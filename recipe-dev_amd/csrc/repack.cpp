// Host-side loader repack: GGUF block bytes <-> the kernel's HBM layout
// (layout.h). Both directions are exact byte permutations (plus the Q8_0 code
// bias and Q4_0 odd-row padding), so unpack(repack(b)) == b.
//
// Reference counterpart: recipe's batch-1 loader interleaves rows four bytes at
// a time across the lanes of a wave (recipe.rs:3162-3212 row_interleave /
// interleave_rows, applied by Buffer::fill_weights at recipe.rs:26980-27010).
// This layout instead gives each lane whole 16-byte parts of one row and makes
// every load instruction of a wave one contiguous 1 KiB run.
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

// One Q6_K scale group (16 weights, codes q[e]) -> words A, B, H (layout.h).
static void q6k_pack_group(const uint8_t* q, uint32_t& A, uint32_t& B, uint32_t& H) {
    A = B = H = 0;
    for (int j = 0; j < 8; ++j) {
        A |= (uint32_t)(q[kQ6EA[j]] & 15) << kQ6NibA[j];
        B |= (uint32_t)(q[kQ6EB[j]] & 15) << kQ6NibB[j];
    }
    for (int e = 0; e < 16; ++e) H |= (uint32_t)((q[e] >> 4) & 3) << kQ6High[e];
}

static void q6k_unpack_group(uint32_t A, uint32_t B, uint32_t H, uint8_t* q) {
    for (int j = 0; j < 8; ++j) {
        q[kQ6EA[j]] = (uint8_t)((A >> kQ6NibA[j]) & 15);
        q[kQ6EB[j]] = (uint8_t)((B >> kQ6NibB[j]) & 15);
    }
    for (int e = 0; e < 16; ++e) q[e] = (uint8_t)(q[e] | (((H >> kQ6High[e]) & 3) << 4));
}

static bool shape_ok(int fmt, int64_t rows, int64_t cols) {
    FormatInfo f = format_info(fmt);
    if (f.block_values == 0 || rows <= 0 || cols <= 0) return false;
    if (cols % f.block_values != 0) return false;
    if (fmt == F16 && cols % 64 != 0) return false;
    return true;
}

int64_t gguf_bytes(int fmt, int64_t rows, int64_t cols) {
    FormatInfo f = format_info(fmt);
    if (!shape_ok(fmt, rows, cols)) return -1;
    return rows * (cols / f.block_values) * f.block_bytes;
}

int repack(int fmt, int64_t rows, int64_t cols, const uint8_t* src, uint8_t* code, uint8_t* meta0, uint8_t* meta1) {
    if (!shape_ok(fmt, rows, cols)) return -1;
    const FormatInfo f = format_info(fmt);
    const RowBytes rb = row_bytes(fmt, cols);
    const int64_t nch = chunks_per_row(fmt, cols);
    const int64_t nblk = cols / f.block_values;
    const int64_t src_row = nblk * f.block_bytes;
    for (int64_t r = 0; r < rows; ++r) {
        const uint8_t* s = src + r * src_row;
        uint8_t* cr = code + r * rb.code;
        uint8_t* m0 = meta0 ? meta0 + r * rb.meta0 : nullptr;
        uint8_t* m1 = meta1 ? meta1 + r * rb.meta1 : nullptr;
        for (int64_t c = 0; c < nch; ++c) {
            switch (fmt) {
                case Q8_0: {
                    const uint8_t* blk = s + c * 34;
                    memcpy(m0 + c * 2, blk, 2);
                    for (int p = 0; p < 2; ++p) {
                        uint8_t* dst = cr + code_offset(c, p, nch, 2);
                        for (int i = 0; i < 16; ++i) dst[i] = (uint8_t)(blk[2 + 16 * p + i] ^ 0x80);
                    }
                    break;
                }
                case Q4_0: {
                    for (int p = 0; p < 2; ++p) {
                        int64_t b = 2 * c + p;
                        uint8_t* dst = cr + code_offset(c, p, nch, 2);
                        if (b < nblk) {
                            const uint8_t* blk = s + b * 18;
                            memcpy(m0 + c * 4 + 2 * p, blk, 2);
                            memcpy(dst, blk + 2, 16);
                        } else {
                            memset(m0 + c * 4 + 2 * p, 0, 2);
                            memset(dst, 0, 16);
                        }
                    }
                    break;
                }
                case Q4_K: {
                    int64_t sb = c / 4;
                    int p = (int)(c % 4);
                    const uint8_t* blk = s + sb * 144;
                    if (p == 0) memcpy(m0 + sb * 16, blk, 16);
                    for (int h = 0; h < 2; ++h) memcpy(cr + code_offset(c, h, nch, 2), blk + 16 + 32 * p + 16 * h, 16);
                    break;
                }
                case Q6_K: {
                    int64_t sb = c / 4;
                    int t = (int)(c % 4);
                    const uint8_t* blk = s + sb * 210;
                    if (t == 0) {
                        memcpy(m0 + sb * 16, blk + 192, 16);
                        memcpy(m1 + sb * 2, blk + 208, 2);
                    }
                    uint32_t lo[8], hi[4];
                    for (int g = 0; g < 4; ++g) {
                        uint8_t q[16];
                        for (int e = 0; e < 16; ++e) q[e] = q6_code(blk, 64 * t + 16 * g + e);
                        q6k_pack_group(q, lo[2 * g], lo[2 * g + 1], hi[g]);
                    }
                    memcpy(cr + code_offset(c, 0, nch, 3), lo, 16);
                    memcpy(cr + code_offset(c, 1, nch, 3), lo + 4, 16);
                    memcpy(cr + code_offset(c, 2, nch, 3), hi, 16);
                    break;
                }
                case F16: {
                    for (int p = 0; p < 8; ++p) memcpy(cr + code_offset(c, p, nch, 8), s + c * 128 + 16 * p, 16);
                    break;
                }
                default: return -1;
            }
        }
    }
    return 0;
}

int unpack(int fmt, int64_t rows, int64_t cols, const uint8_t* code, const uint8_t* meta0, const uint8_t* meta1,
           uint8_t* dst) {
    if (!shape_ok(fmt, rows, cols)) return -1;
    const FormatInfo f = format_info(fmt);
    const RowBytes rb = row_bytes(fmt, cols);
    const int64_t nch = chunks_per_row(fmt, cols);
    const int64_t nblk = cols / f.block_values;
    const int64_t dst_row = nblk * f.block_bytes;
    for (int64_t r = 0; r < rows; ++r) {
        uint8_t* d = dst + r * dst_row;
        const uint8_t* cr = code + r * rb.code;
        const uint8_t* m0 = meta0 ? meta0 + r * rb.meta0 : nullptr;
        const uint8_t* m1 = meta1 ? meta1 + r * rb.meta1 : nullptr;
        for (int64_t c = 0; c < nch; ++c) {
            switch (fmt) {
                case Q8_0: {
                    uint8_t* blk = d + c * 34;
                    memcpy(blk, m0 + c * 2, 2);
                    for (int p = 0; p < 2; ++p) {
                        const uint8_t* src = cr + code_offset(c, p, nch, 2);
                        for (int i = 0; i < 16; ++i) blk[2 + 16 * p + i] = (uint8_t)(src[i] ^ 0x80);
                    }
                    break;
                }
                case Q4_0: {
                    for (int p = 0; p < 2; ++p) {
                        int64_t b = 2 * c + p;
                        if (b >= nblk) continue;
                        uint8_t* blk = d + b * 18;
                        memcpy(blk, m0 + c * 4 + 2 * p, 2);
                        memcpy(blk + 2, cr + code_offset(c, p, nch, 2), 16);
                    }
                    break;
                }
                case Q4_K: {
                    int64_t sb = c / 4;
                    int p = (int)(c % 4);
                    uint8_t* blk = d + sb * 144;
                    if (p == 0) memcpy(blk, m0 + sb * 16, 16);
                    for (int h = 0; h < 2; ++h) memcpy(blk + 16 + 32 * p + 16 * h, cr + code_offset(c, h, nch, 2), 16);
                    break;
                }
                case Q6_K: {
                    int64_t sb = c / 4;
                    int t = (int)(c % 4);
                    uint8_t* blk = d + sb * 210;
                    if (t == 0) {
                        memset(blk, 0, 192);
                        memcpy(blk + 192, m0 + sb * 16, 16);
                        memcpy(blk + 208, m1 + sb * 2, 2);
                    }
                    uint32_t lo[8], hi[4];
                    memcpy(lo, cr + code_offset(c, 0, nch, 3), 16);
                    memcpy(lo + 4, cr + code_offset(c, 1, nch, 3), 16);
                    memcpy(hi, cr + code_offset(c, 2, nch, 3), 16);
                    for (int g = 0; g < 4; ++g) {
                        uint8_t q[16];
                        q6k_unpack_group(lo[2 * g], lo[2 * g + 1], hi[g], q);
                        for (int e = 0; e < 16; ++e) q6_store(blk, 64 * t + 16 * g + e, q[e]);
                    }
                    break;
                }
                case F16: {
                    for (int p = 0; p < 8; ++p) memcpy(d + c * 128 + 16 * p, cr + code_offset(c, p, nch, 8), 16);
                    break;
                }
                default: return -1;
            }
        }
    }
    return 0;
}

}  // namespace rq
