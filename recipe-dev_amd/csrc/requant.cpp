// Host requantization to Q8_0: the storage recipe's int(8) profile gives a
// bound weight whose format it does not keep (finish_int_sums and
// requantize_bound, recipe.rs:22327-22437: Q4_K and Q8_0 stay, every other
// single-format weight becomes Q8_0), encoded as recipe's device quantizer
// encodes it (emit_requantize, DeviceQuantizer::Q8_0, recipe.rs:8016-8080).
// Per 32 decoded values: the first value of largest magnitude e, scale =
// |e| / 127, inverse = 1 / scale (0 for a zero scale), code = trunc(v * inverse
// +- 0.5) clamped to [-128, 127] (the +-0.5 an fp32 sum, as recipe adds it),
// d = the scale rounded half to even to fp16. Every step is one fp32
// operation, and this file is built without contraction, so the bytes are the
// ones recipe's load kernel writes.
#include "requant.h"

#include <math.h>
#include <string.h>

#pragma clang fp contract(off)

namespace rq {

namespace {

float half_value(const uint8_t* p) {
    _Float16 h;
    memcpy(&h, p, 2);
    return (float)h;
}

// Value i of a block, exact in fp32 for these formats.
float decode(int fmt, const uint8_t* blk, int i) {
    switch (fmt) {
        case F16: return half_value(blk);
        case Q8_0: return (float)(int8_t)blk[2 + i] * half_value(blk);
        case Q4_0: return (float)((int)((blk[2 + (i & 15)] >> (4 * (i >> 4))) & 15) - 8) * half_value(blk);
        case Q6_K: {
            const int chunk = i / 128, local = (i % 128) / 32, within = i % 32;
            const int lo = (blk[chunk * 64 + within + 32 * (local & 1)] >> (4 * (local >> 1))) & 15;
            const int hi = (blk[128 + chunk * 32 + within] >> (2 * local)) & 3;
            const int sc = (int8_t)blk[192 + i / 16];
            return half_value(blk + 208) * (float)(sc * ((lo | (hi << 4)) - 32));
        }
        default: return NAN;
    }
}

}  // namespace

bool requantizable_to_q8_0(int fmt) { return fmt == F16 || fmt == Q8_0 || fmt == Q4_0 || fmt == Q6_K; }

int requantize_q8_0(int fmt, int64_t rows, int64_t cols, const uint8_t* src, uint8_t* dst) {
    const FormatInfo f = format_info(fmt);
    if (!requantizable_to_q8_0(fmt) || rows <= 0 || cols <= 0 || cols % 32 != 0 || cols % f.block_values != 0)
        return -1;
    const int64_t row_src = cols / f.block_values * f.block_bytes;
    for (int64_t r = 0; r < rows; ++r) {
        const uint8_t* row = src + r * row_src;
        for (int64_t b = 0; b < cols / 32; ++b) {
            float v[32];
            for (int i = 0; i < 32; ++i) {
                const int64_t k = b * 32 + i;
                v[i] = decode(fmt, row + (k / f.block_values) * f.block_bytes, (int)(k % f.block_values));
            }
            float e = 0.f;
            for (int i = 0; i < 32; ++i)
                if (fabsf(v[i]) > fabsf(e)) e = v[i];
            const float scale = fabsf(e) / 127.f;
            const float inverse = scale == 0.f ? 0.f : 1.f / scale;
            uint8_t* blk = dst + (r * (cols / 32) + b) * 34;
            const _Float16 d = (_Float16)scale;
            memcpy(blk, &d, 2);
            for (int i = 0; i < 32; ++i) {
                const float q = v[i] * inverse;
                const float rounded = q >= 0.f ? q + 0.5f : q + -0.5f;
                int c = (int)rounded;
                c = c < -128 ? -128 : (c > 127 ? 127 : c);
                blk[2 + i] = (uint8_t)(int8_t)c;
            }
        }
    }
    return 0;
}

}  // namespace rq
