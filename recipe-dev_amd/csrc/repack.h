// Host-side loader repack between GGUF block bytes and the kernel layout.
#pragma once

#include "layout.h"

namespace rq {

// Bytes of `rows` x `cols` weights as GGUF stores them; -1 on a bad shape.
int64_t gguf_bytes(int fmt, int64_t rows, int64_t cols);

// GGUF rows -> code plane + meta planes (sizes from row_bytes() * rows).
int repack(int fmt, int64_t rows, int64_t cols, const uint8_t* src, uint8_t* code, uint8_t* meta0, uint8_t* meta1);

// The inverse of repack().
int unpack(int fmt, int64_t rows, int64_t cols, const uint8_t* code, const uint8_t* meta0, const uint8_t* meta1,
           uint8_t* dst);

}  // namespace rq
