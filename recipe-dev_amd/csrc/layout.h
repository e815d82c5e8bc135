// Repacked HBM layout of GGUF block weights for the gfx950 matrix-vector
// kernels. Shared by host code (repack, unpack) and device code (kernels).
//
// A row of K weights is cut into "chunks": the unit one lane decodes per step.
// Each chunk's quantized codes occupy QP 16-byte parts in the code plane; the
// per-block scales live in one or two small meta planes. Within a row, chunks
// are grouped 64 at a time and the parts of a group are stored part-major:
//
//     group B of a row (nb = min(64, chunks - 64*B) chunks):
//         part 0 of chunks 0..nb-1, part 1 of chunks 0..nb-1, ...
//
// so the 64 lanes of a wave that take 64 consecutive chunks read one
// contiguous 1 KiB run per load instruction (16 B per lane). Group B starts at
// 64*B*QP*16 bytes into the row, which keeps every row a contiguous stream.
//
// Per format (GGML type id, recipe.rs:9925-9961; block sizes recipe.rs:15811-15826):
//   Q8_0 (8)   chunk = 1 block (32 w). Codes stored as unsigned q+128 (byte ^ 0x80),
//              2 parts. meta0 = fp16 d per chunk.
//   Q4_0 (2)   chunk = 2 blocks (64 w). Part p = the 16 code bytes of block 2c+p,
//              unchanged. meta0 = the two fp16 d per chunk (4 B). A row with an
//              odd block count gets one zero block (d = 0) at its end.
//   Q4_K (12)  chunk = a pair of 32-w sub-blocks (64 w, code bytes 32p..32p+31 of
//              the superblock, unchanged), 2 parts. meta0 = the superblock's first
//              16 bytes (d, dmin, 12 bytes of 6-bit scales/mins), unchanged.
//   Q6_K (14)  chunk = a quarter superblock (64 w), 3 parts: two parts of low
//              nibbles and one of high 2-bit fields, re-arranged per 16-weight
//              scale group as described at q6k_pack_group(). meta0 = the 16 int8
//              scales per superblock, meta1 = fp16 d per superblock.
//   F16 (1)    chunk = 64 halves, 8 parts. No meta.
//   F32 (0)    not repacked here (the kernels take fp16/fp32 activations and
//              quantized or f16 weights).
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
    int meta0_per_row_unit;  // bytes of meta0 per chunk (or per superblock, see below)
    int meta0_per_superblock;  // 1 if meta0 is per superblock, 0 if per chunk
    int meta1_bytes;    // bytes of meta1 per superblock (0 = none)
    int sums;           // activation sums per chunk the f16 kernels need
};

RQ_HD FormatInfo format_info(int fmt) {
    switch (fmt) {
        case Q8_0: return FormatInfo{32, 34, 32, 2, 2, 0, 0, 1};
        case Q4_0: return FormatInfo{32, 18, 64, 2, 4, 0, 0, 4};
        case Q4_K: return FormatInfo{256, 144, 64, 2, 16, 1, 0, 2};
        case Q6_K: return FormatInfo{256, 210, 64, 3, 16, 1, 2, 8};
        case F16: return FormatInfo{1, 2, 64, 8, 0, 0, 0, 0};
        default: return FormatInfo{0, 0, 0, 0, 0, 0, 0, 0};
    }
}

RQ_HD bool format_supported(int fmt) { return format_info(fmt).block_values != 0; }

// Chunks per row of `cols` weights (Q4_0 rounds an odd block count up).
RQ_HD int64_t chunks_per_row(int fmt, int64_t cols) {
    FormatInfo f = format_info(fmt);
    return (cols + f.chunk_values - 1) / f.chunk_values;
}

// Byte offset of part `part` of chunk `c` within a row of `nch` chunks.
RQ_HD int64_t code_offset(int64_t c, int part, int64_t nch, int parts) {
    int64_t group = c >> 6;
    int64_t within = c & 63;
    int64_t nb = nch - (group << 6);
    if (nb > 64) nb = 64;
    return group * 64 * parts * 16 + ((int64_t)part * nb + within) * 16;
}

// Bytes of one row in each plane.
struct RowBytes {
    int64_t code, meta0, meta1;
};

RQ_HD RowBytes row_bytes(int fmt, int64_t cols) {
    FormatInfo f = format_info(fmt);
    int64_t nch = chunks_per_row(fmt, cols);
    RowBytes r;
    r.code = nch * f.code_parts * 16;
    if (f.meta0_per_superblock)
        r.meta0 = (cols / f.block_values) * f.meta0_per_row_unit;
    else
        r.meta0 = nch * f.meta0_per_row_unit;
    r.meta1 = f.meta1_bytes ? (cols / f.block_values) * f.meta1_bytes : 0;
    return r;
}

// Q6_K: the 16 weights e = 0..15 of one scale group become two code words A, B
// (low nibbles) and one word H (high 2-bit fields) so that one mask-and-or per
// pair builds two fp16 values 1024 + q (x1 pairs) or 1024 + 16 q (x16 pairs):
//   A: e0@0 e1@16 e2@8 e3@24 (x1 nibbles)   e8@4 e9@20 e10@12 e11@28 (x16 nibbles)
//   B: e4@0 e5@16 e6@8 e7@24                e12@4 e13@20 e14@12 e15@28
//   H (2-bit fields): e0@4 e1@20 e8@8 e9@24 e2@6 e3@22 e10@10 e11@26
//                     e4@12 e5@28 e12@16 e13@0 e6@14 e7@30 e14@18 e15@2
// Read back with H, H>>2, rotr(H,8) and rotr(H,10) for A lo, A hi, B lo, B hi.
static const int kQ6NibA[8] = {0, 16, 8, 24, 4, 20, 12, 28};  // e0,e1,e2,e3,e8,e9,e10,e11
static const int kQ6NibB[8] = {0, 16, 8, 24, 4, 20, 12, 28};  // e4,e5,e6,e7,e12,e13,e14,e15
static const int kQ6EA[8] = {0, 1, 2, 3, 8, 9, 10, 11};
static const int kQ6EB[8] = {4, 5, 6, 7, 12, 13, 14, 15};
static const int kQ6High[16] = {4, 20, 6, 22, 12, 28, 14, 30, 8, 24, 10, 26, 16, 0, 18, 2};  // by e

}  // namespace rq
