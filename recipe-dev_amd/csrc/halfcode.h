// Exact fp16 forms of quantized weight codes, shared by the matrix-core
// kernels and the fp16-activation vector kernel. Every code (q, q - 8,
// l + 16h - 32, an int8) is a small integer, exact in fp16, so products with
// fp16 activations are exact and only the accumulation rounds.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rq {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef _Float16 hv2_t __attribute__((ext_vector_type(2)));
typedef float f4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t pk_add_h(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(hv2_t, a) + __builtin_bit_cast(hv2_t, b));
}

// Eight 4-bit codes u (weight i in bits 4i..4i+3) -> four words of fp16 pairs
// (u_2t - off, u_2t+1 - off). The even code goes into the mantissa of 1024.0
// (0x6400 | u), the odd one, left in its byte's high nibble, into the mantissa
// of 64.0 (0x5400 | 16u), and one packed fp16 add of (-1024 - off, -64 - off)
// removes both offsets exactly.
__device__ __forceinline__ void nibbles_to_h(uint32_t w, uint32_t neg, uint32_t (&o)[4]) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const uint32_t sel = (uint32_t)t | 0x0c00u | ((uint32_t)t << 16) | 0x0c000000u;
        const uint32_t b = __builtin_amdgcn_perm(0u, w, sel);  // [byte t, 0, byte t, 0]
        o[t] = pk_add_h((b & 0x00F0000Fu) | 0x54006400u, neg);
    }
}

// Four int8 codes -> two words of fp16 pairs: q + 128 in the mantissa of
// 1024.0, then - 1152.
__device__ __forceinline__ void bytes_to_h(uint32_t w, uint32_t& o0, uint32_t& o1) {
    const uint32_t u = w ^ 0x80808080u;
    const uint32_t neg = 0xE480E480u;  // (-1152, -1152)
    o0 = pk_add_h(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u), neg);
    o1 = pk_add_h(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u), neg);
}

// Q6_K: eight low nibbles L (codes already un-XORed) and their high fields
// as nibbles Hx -> four words of fp16 pairs (l + 16h - 32).
__device__ __forceinline__ void q6_to_h(uint32_t L, uint32_t Hx, uint32_t (&o)[4]) {
    const uint32_t ev = (L & 0x0F0F0F0Fu) | ((Hx & 0x03030303u) << 4);   // byte t: code of weight 2t
    const uint32_t od = ((L >> 4) & 0x0F0F0F0Fu) | (Hx & 0x30303030u);   // byte t: code of weight 2t+1
    const uint32_t neg = 0xE420E420u;  // (-1056, -1056)
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const uint32_t sel = (uint32_t)t | 0x0c00u | ((uint32_t)(4 + t) << 16) | 0x0c000000u;
        o[t] = pk_add_h(__builtin_amdgcn_perm(od, ev, sel) | 0x64006400u, neg);
    }
}

}  // namespace rq
