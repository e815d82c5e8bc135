// recipe's scalar activations on the device, in fp32.
//
// The programs of activation_program (recipe.rs:22579-22727) with the default
// constants of recipe's build (Cargo.toml:117-124): leak slope 0.01, ELU
// alpha 1, SELU alpha 1.6732632423543772 and scale 1.0507009873554805, GELU
// scale sqrt(2/pi) and cubic 0.044715, Huber threshold 1. Codes are
// Activation::code() (recipe.rs:13925-13950); kActGeluFp16 is Gelu as the
// llama.cpp profile's gelu table runs it (the input and the result rounded to
// fp16 inside [-10, 10], the input itself above 10, zero below -10). `factor` is Scale's constant and PReLU's slope.
#pragma once

#include <hip/hip_runtime.h>

namespace rq {

enum ActCode : int {
    kActLinear = 0, kActCos = 1, kActExp = 2, kActLog = 3, kActLn = 4, kActHuber = 5, kActTan = 6, kActRelu = 7,
    kActLeak = 8, kActSigmoid = 9, kActTanh = 10, kActSelu = 11, kActGelu = 12, kActSilu = 13, kActElu = 14,
    kActPrelu = 15, kActScale = 16, kActSqrt = 17, kActSoftplus = 18, kActGeluFp16 = 32
};

inline bool act_known(int code) { return (code >= 0 && code <= 18) || code == kActGeluFp16; }

// 0.5 (tanh(v / 2) + 1): recipe's Sigmoid (and SiLU's gate), recipe.rs:22662-22668.
__device__ __forceinline__ float act_sigmoid_tanh(float v) { return 0.5f * (tanhf(0.5f * v) + 1.0f); }

__device__ __forceinline__ float act_gelu_tanh(float v) {
    return (0.5f * v) * (1.0f + tanhf((0.7978845608028654f * v) * fmaf(0.044715f * v, v, 1.0f)));
}

__device__ inline float act_apply(int code, float factor, float x) {
    const bool positive = x > 0.f;
    switch (code) {
        case kActLinear: return x;
        case kActCos: return cosf(x);
        case kActExp: return expf(x);
        case kActSqrt: return sqrtf(x);
        case kActSoftplus: return (positive ? x : 0.f) + logf(1.0f + expf(0.f - fabsf(x)));
        case kActLog:
        case kActLn: {
            const float magnitude = logf(1.0f + fabsf(x));
            const float s = positive ? magnitude : 0.f - magnitude;
            return code == kActLog ? s / 2.302585092994045684f : s;
        }
        case kActHuber: {
            const float a = fabsf(x);
            return a > 1.0f ? 1.0f * (a - 0.5f * 1.0f) : 0.5f * (x * x);
        }
        case kActTan: return sinf(x) / cosf(x);
        case kActRelu: return positive ? x : 0.f;
        case kActLeak: return positive ? x : 0.01f * x;
        case kActPrelu: return positive ? x : factor * x;
        case kActElu: return positive ? x : 1.0f * (expf(positive ? 0.f : x) - 1.0f);
        case kActSelu: return 1.0507009873554805f * (positive ? x : 1.6732632423543772f * (expf(positive ? 0.f : x) - 1.0f));
        case kActSigmoid: return act_sigmoid_tanh(x);
        case kActSilu: return x * act_sigmoid_tanh(x);
        case kActTanh: return tanhf(x);
        case kActGelu: return act_gelu_tanh(x);
        case kActGeluFp16: {
            if (x > 10.f) return x;
            if (x < -10.f) return 0.f;
            const float h = (float)(_Float16)x;
            return (float)(_Float16)act_gelu_tanh(h);
        }
        case kActScale: return factor * x;
        default: return __builtin_nanf("");
    }
}

// act_apply with SiLU (llama-style experts) inline and the rest out of the
// hot path's layout.
__device__ __forceinline__ float act_apply_likely_silu(int code, float factor, float x) {
    if (__builtin_expect(code == kActSilu, 1)) return x * act_sigmoid_tanh(x);
    return act_apply(code, factor, x);
}

// act_apply with Sigmoid (the usual shared-expert gate) inline.
__device__ __forceinline__ float act_apply_likely_sigmoid(int code, float factor, float x) {
    if (__builtin_expect(code == kActSigmoid, 1)) return act_sigmoid_tanh(x);
    return act_apply(code, factor, x);
}

}  // namespace rq
