// Host requantization of block weights to Q8_0 as recipe's int(8) profile
// stores them (requant.cpp).
#pragma once

#include "layout.h"

namespace rq {

// F16, Q8_0, Q4_0 and Q6_K decode exactly in fp32 and can be re-encoded.
bool requantizable_to_q8_0(int fmt);

// rows x cols GGUF weights of `fmt` -> rows * cols / 32 Q8_0 blocks at dst.
// Returns 0, or -1 for an unsupported format or shape.
int requantize_q8_0(int fmt, int64_t rows, int64_t cols, const uint8_t* src, uint8_t* dst);

}  // namespace rq
