// Repacked HBM layout of GGUF block weights for the gfx950 matrix-vector
// kernels. Shared by host code (repack, unpack) and device code (kernels).
//
// A row of K weights is cut into "chunks": the unit one lane decodes per step.
// Chunks are grouped 64 at a time; a group of nb chunks (64, or fewer in a
// row's last group) is stored as its QP 16-byte code parts, part-major, then
// the group's scale bytes:
//
//     part 0 of chunks 0..nb-1 | part 1 of chunks 0..nb-1 | ... | meta of the group
//
// so the 64 lanes of a wave that take 64 consecutive chunks read one
// contiguous 1 KiB run per load instruction (16 bytes per lane), and a row is
// one contiguous stream with its scales beside its codes. Rows start 16-byte
// aligned (a row's bytes round up to a multiple of 16, or of 128 from 4 KiB).
//
// Per format (GGML type id, recipe.rs:9925-9961; block sizes recipe.rs:15811-15826).
// Four-bit codes are stored in natural weight order, two per byte (weight 2j
// in the low nibble of byte j, weight 2j+1 in the high nibble), each XOR 8, so
// that a signed 4-bit read of the nibble is q - 8 and v_dot8_i32_i4 takes eight
// weights from one word with no unpacking:
//   Q8_0 (8)   chunk = 1 block (32 w), 2 parts: the 32 int8 codes unchanged.
//              meta0 = fp16 d per chunk.
//   Q4_0 (2)   chunk = 2 blocks (64 w); part p = block 2c+p's 32 codes as above.
//              meta0 = the two fp16 d per chunk (4 B). A row with an odd block
//              count gets one zero block (d = 0) at its end.
//   Q4_K (12)  chunk = the sub-block pair 2p, 2p+1 of a superblock (64 w); part j =
//              sub-block 2p+j's 32 codes as above. meta0 = the superblock's d and
//              dmin, then its 16 six-bit scales and minimums as four 24-bit
//              fields, chunk p's at bit 24p (scale 2p, min 2p, scale 2p+1,
//              min 2p+1): the k_scale bytes' 96 bits, reordered (repack.cpp).
//   Q6_K (14)  chunk = a quarter superblock (64 w), 3 parts: parts 0-1 hold the
//              64 low nibbles l as above; part 2 holds one word per 16-weight
//              scale group g whose bits 4j..4j+1 are the high field h of weight
//              16g+j and bits 4j+2..4j+3 that of weight 16g+8+j (j < 8), so that
//              H & 0x33333333 and (H >> 2) & 0x33333333 are nibble words of h in
//              natural order. meta0 = the 16 int8 scales per superblock, meta1 =
//              fp16 d per superblock.
//   F16 (1)    chunk = 64 halves, 8 parts. No meta.
#pragma once

#include <stddef.h>
#include <stdint.h>

#ifdef __HIPCC__
#define RQ_HD __host__ __device__ inline
#else
#define RQ_HD inline
#endif

namespace rq {

enum Format : int { F32 = 0, F16 = 1, Q4_0 = 2, Q8_0 = 8, Q4_K = 12, Q6_K = 14 };

struct FormatInfo {
    int block_values;   // weights per GGUF block
    int block_bytes;    // bytes per GGUF block
    int chunk_values;   // weights per chunk
    int code_parts;     // 16-byte code parts per chunk
    int meta_quad;      // scale bytes per 4 chunks
};

RQ_HD FormatInfo format_info(int fmt) {
    switch (fmt) {
        case Q8_0: return FormatInfo{32, 34, 32, 2, 8};    // 4 x fp16 d
        case Q4_0: return FormatInfo{32, 18, 64, 2, 16};   // 8 x fp16 d
        case Q4_K: return FormatInfo{256, 144, 64, 2, 16}; // one superblock's d, dmin, scales
        case Q6_K: return FormatInfo{256, 210, 64, 3, 18}; // 16 int8 scales + fp16 d
        case F16: return FormatInfo{1, 2, 64, 8, 0};
        default: return FormatInfo{0, 0, 0, 0, 0};
    }
}

RQ_HD bool format_supported(int fmt) { return format_info(fmt).block_values != 0; }

// Chunks per row of `cols` weights (Q4_0 rounds an odd block count up).
RQ_HD int64_t chunks_per_row(int fmt, int64_t cols) {
    FormatInfo f = format_info(fmt);
    return (cols + f.chunk_values - 1) / f.chunk_values;
}

// Bytes of a group of nb chunks (nb a multiple of 4 except in Q8_0 and Q4_0
// last groups, whose meta is per chunk).
RQ_HD int64_t group_bytes(const FormatInfo& f, int64_t nb) {
    return nb * f.code_parts * 16 + (nb * f.meta_quad + 3) / 4;
}

// Bytes of one row: its groups rounded up to 16, and rows of 4 KiB or more
// to whole 128-byte lines, so that no cache line holds the end of one such
// row and the start of the next (different workgroups read the two rows at
// different times, and the line would come from HBM twice: Q6_K rows of 5120
// weights, 4,200 bytes, read 15 % of their bytes twice); shorter rows keep
// the 16-byte rounding, where a line's padding would be a larger share.
RQ_HD int64_t row_bytes(int fmt, int64_t cols) {
    const FormatInfo f = format_info(fmt);
    const int64_t nch = chunks_per_row(fmt, cols);
    const int64_t full = nch / 64, rest = nch % 64;
    const int64_t b = full * group_bytes(f, 64) + (rest ? group_bytes(f, rest) : 0);
    const int64_t b16 = (b + 15) / 16 * 16;
    return b16 >= 4096 ? (b16 + 127) / 128 * 128 : b16;
}

// Where chunk c of a row of nch chunks lives: its group's start, the group's
// chunk count and the chunk's index in it.
struct ChunkPlace {
    int64_t group_start;
    int nb, within;
};

RQ_HD ChunkPlace chunk_place(int fmt, int64_t c, int64_t nch) {
    const FormatInfo f = format_info(fmt);
    ChunkPlace p;
    const int64_t group = c >> 6;
    const int64_t rest = nch - (group << 6);
    p.nb = (int)(rest > 64 ? 64 : rest);
    p.within = (int)(c & 63);
    p.group_start = group * group_bytes(f, 64);
    return p;
}

// Byte offset, within its row, of code part `part` of chunk c.
RQ_HD int64_t code_offset(int fmt, int64_t c, int part, int64_t nch) {
    const ChunkPlace p = chunk_place(fmt, c, nch);
    return p.group_start + ((int64_t)part * p.nb + p.within) * 16;
}

// Byte offset, within its row, of the group meta region holding chunk c.
RQ_HD int64_t meta_offset(int fmt, int64_t c, int64_t nch) {
    const ChunkPlace p = chunk_place(fmt, c, nch);
    return p.group_start + (int64_t)format_info(fmt).code_parts * p.nb * 16;
}

}  // namespace rq
