// Host-side loader repack between GGUF block bytes and the kernel layout.
#pragma once

#include "layout.h"

namespace rq {

// Bytes of `rows` x `cols` weights as GGUF stores them; -1 on a bad shape.
int64_t gguf_bytes(int fmt, int64_t rows, int64_t cols);

// Bytes of the repacked layout (rows * row_bytes); -1 on a bad shape.
int64_t layout_bytes(int fmt, int64_t rows, int64_t cols);

// GGUF rows -> the repacked layout (layout_bytes(...) bytes at dst).
int repack(int fmt, int64_t rows, int64_t cols, const uint8_t* src, uint8_t* dst);

// The inverse of repack().
int unpack(int fmt, int64_t rows, int64_t cols, const uint8_t* src, uint8_t* dst);

}  // namespace rq
