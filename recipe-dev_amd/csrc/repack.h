// Host-side loader repack between GGUF block bytes and the kernel layout.
#pragma once

#include "layout.h"

namespace rq {

// Largest shape a weight may have: row indices are 32-bit in the kernels.
constexpr int64_t kMaxRows = 0x7fffffff;
constexpr int64_t kMaxCols = int64_t(1) << 30;

// Bytes of `rows` x `cols` weights as GGUF stores them; -1 on a bad shape
// (rows or cols out of range, or a size that does not fit in 63 bits).
int64_t gguf_bytes(int fmt, int64_t rows, int64_t cols);

// Bytes of the repacked layout (rows * row_bytes); -1 on a bad shape, as above.
int64_t layout_bytes(int fmt, int64_t rows, int64_t cols);

// GGUF rows -> the repacked layout (layout_bytes(...) bytes at dst).
int repack(int fmt, int64_t rows, int64_t cols, const uint8_t* src, uint8_t* dst);

// The inverse of repack().
int unpack(int fmt, int64_t rows, int64_t cols, const uint8_t* src, uint8_t* dst);

}  // namespace rq
