// Kernels around the projections of a single-token decode step, so that a
// whole decoder layer runs on the device between the quantized products:
// residual add + RMSNorm, NeoX rotary embedding with the fp16 KV-cache append,
// grouped-query attention over the cache, SiLU-GLU, the argmax of the logits
// and the next token's embedding row. They follow recipe's lowering of an attention block
// (lower_attention, recipe.rs:23056-23150: one QKV projection laid out
// queries, keys, values; rotary on queries and keys; scores scaled by
// 1/sqrt(head width); softmax; the output projection) and of the
// feed-forward (silu(gate) * up, recipe.rs:23279-23286, 22662-22668).
// Activations are fp32 (recipe's state precision); the cache is fp16.
#include <hip/hip_runtime.h>
#include <math.h>

#include "decode.h"
#include "stage.h"

namespace rq {

// ------------------------------------------------------------ RMSNorm ----

// x += delta (when given); out = x / sqrt(mean(x^2) + eps) * w. One workgroup;
// the sum of squares is taken in a fixed order (per-thread parts, then a tree
// of fixed pairs), so the result does not depend on scheduling.
__global__ void __launch_bounds__(1024) add_rmsnorm_kernel(float* x, const float* delta, const float* w, int n,
                                                            float eps, float* out) {
    __shared__ float part[1024];
    const int t = threadIdx.x;
    float ss = 0.f;
    for (int i = t; i < n; i += blockDim.x) {
        float v = x[i];
        if (delta) {
            v += delta[i];
            x[i] = v;
        }
        ss = fmaf(v, v, ss);
    }
    part[t] = ss;
    __syncthreads();
    // tree over the parts in a fixed pairing
    for (int s = blockDim.x / 2; s > 0; s >>= 1) {
        if (t < s) part[t] += part[t + s];
        __syncthreads();
    }
    const float scale = 1.0f / sqrtf(part[0] / (float)n + eps);
    for (int i = t; i < n; i += blockDim.x) out[i] = x[i] * scale * w[i];
}

// ------------------------------------------------------------- rotary ----

// NeoX rotary (rope_pair, amd-nv-cpu.ll:3719-3780 without yarn): pair i of a
// head, (x_i, x_{i + half}), turns by pos * base^(-2i/dims). The angle and
// its sine and cosine are taken in f64, the rotation in fp32. Queries and keys
// rotate in place in `qkv` ([q heads | k heads | v heads] x head_dim); the
// rotated keys and the values are appended to the caches at `pos`
// (layout [kv head][position][head_dim], fp16).
__global__ void __launch_bounds__(256) rope_kv_kernel(float* qkv, const int* pos_dev, int nq, int nkv, int hd,
                                                      double base, __half* kc, __half* vc, int max_ctx) {
    const int pos = *pos_dev;
    const int half = hd / 2;
    const int pairs = (nq + nkv) * half;
    const double lb = log(base);
    for (int p = blockIdx.x * blockDim.x + threadIdx.x; p < pairs; p += gridDim.x * blockDim.x) {
        const int head = p / half, i = p % half;
        const double angle = (double)pos * exp(-((double)(2 * i) / (double)hd) * lb);
        const float c = (float)cos(angle), s = (float)sin(angle);
        float* h = qkv + (size_t)head * hd;
        const float a = h[i], b = h[i + half];
        const float ra = a * c - b * s, rb = b * c + a * s;
        h[i] = ra;
        h[i + half] = rb;
        if (head >= nq && pos >= 0 && pos < max_ctx) {  // a key head: append it (rotated) and its value head
            const int kh = head - nq;
            __half* kdst = kc + ((size_t)kh * max_ctx + pos) * hd;
            kdst[i] = __float2half(ra);
            kdst[i + half] = __float2half(rb);
            const float* vsrc = qkv + (size_t)(nq + nkv + kh) * hd;
            __half* vdst = vc + ((size_t)kh * max_ctx + pos) * hd;
            vdst[i] = __float2half(vsrc[i]);
            vdst[i + half] = __float2half(vsrc[i + half]);
        }
    }
}

// ---------------------------------------------------------- attention ----

// One workgroup per (kv head, chunk of kAttnChunk positions). Pass 1: the
// scores of every query head of the group against every position of the chunk
// (eight lanes per position, head_dim / 8 values each, summed over the eight
// lanes), scaled by 1/sqrt(head_dim), into LDS. Pass 2: per query head the
// chunk's maximum m, the weights e_t = exp(s_t - m) and their sum l. Pass 3:
// o[d] = sum_t e_t v_t[d]. The chunk's (m, l, o) go to the workspace and
// attn_combine_kernel merges the chunks.
constexpr int kAttnChunk = 128;
constexpr int kAttnMaxGroup = 8;     // query heads per kv head
constexpr int kAttnMaxHead = 256;    // head_dim

__device__ __forceinline__ float sum8(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xf, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xf, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xf, 0xf, false));
    return v;  // every lane of the aligned group of eight holds the sum
}

__global__ void __launch_bounds__(256) attn_partial_kernel(const float* q, const __half* kc, const __half* vc,
                                                           const int* pos_dev, int nq, int nkv, int hd, int max_ctx,
                                                           float scale, float* part_ml, float* part_o) {
    __shared__ float sc[kAttnMaxGroup][kAttnChunk];
    __shared__ float ml[kAttnMaxGroup][2];
    __shared__ float sq[kAttnMaxGroup * kAttnMaxHead];
    const int kh = blockIdx.x, chunk = blockIdx.y;
    const int len = min(*pos_dev + 1, max_ctx);  // positions past the cache are not read
    const int t0 = chunk * kAttnChunk;
    const int group = nq / nkv;
    const int t = threadIdx.x;
    const int per = hd / 8;  // values per lane in pass 1 (a multiple of 8)
    const __half* kbase = kc + (size_t)kh * max_ctx * hd;
    const __half* vbase = vc + (size_t)kh * max_ctx * hd;
    for (int i = t; i < group * hd; i += blockDim.x) sq[i] = q[(size_t)kh * group * hd + i];
    __syncthreads();
    // pass 1: eight lanes per position, 32 positions per sweep of 256 threads
    const int sub = t & 7, slot = t >> 3;
    for (int p0 = 0; p0 < kAttnChunk; p0 += 32) {
        const int tp = t0 + p0 + slot;
        float dots[kAttnMaxGroup];
#pragma unroll
        for (int g = 0; g < kAttnMaxGroup; ++g) dots[g] = 0.f;
        if (tp < len) {
            const uint4* krow = reinterpret_cast<const uint4*>(kbase + (size_t)tp * hd + sub * per);
            for (int e8 = 0; e8 < per / 8; ++e8) {
                const uint4 raw = krow[e8];
                const uint32_t w4[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
                for (int h2 = 0; h2 < 4; ++h2) {
                    const int e = e8 * 8 + 2 * h2;
                    const float k0 = half_lo(w4[h2]), k1 = half_hi(w4[h2]);
#pragma unroll
                    for (int g = 0; g < kAttnMaxGroup; ++g)
                        if (g < group) {
                            const float* qg = sq + g * hd + sub * per + e;
                            dots[g] = fmaf(qg[1], k1, fmaf(qg[0], k0, dots[g]));
                        }
                }
            }
        }
#pragma unroll
        for (int g = 0; g < kAttnMaxGroup; ++g) {
            const float s = sum8(dots[g]);
            if (g < group && sub == 0) sc[g][p0 + slot] = tp < len ? s * scale : -INFINITY;
        }
    }
    __syncthreads();
    // pass 2: one wave per query head of the group (up to four at a time)
    const int lane = t & 63, wave = t >> 6;
    for (int g = wave; g < group; g += 4) {
        float m = -INFINITY;
        for (int i = lane; i < kAttnChunk; i += 64) m = fmaxf(m, sc[g][i]);
        for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
        float l = 0.f;
        for (int i = lane; i < kAttnChunk; i += 64) {
            const float e = sc[g][i] == -INFINITY ? 0.f : expf(sc[g][i] - m);
            sc[g][i] = e;
            l += e;
        }
        for (int off = 32; off > 0; off >>= 1) l += __shfl_xor(l, off);
        if (lane == 0) {
            ml[g][0] = m;
            ml[g][1] = l;
        }
    }
    __syncthreads();
    // pass 3: thread d (and d + 256, ...) accumulates o[g][d] for every head of the group
    const int n_out = hd;
    for (int d = t; d < n_out; d += blockDim.x) {
        float o[kAttnMaxGroup];
#pragma unroll
        for (int g = 0; g < kAttnMaxGroup; ++g) o[g] = 0.f;
        const int tn = len - t0 < kAttnChunk ? len - t0 : kAttnChunk;
        for (int i = 0; i < tn; ++i) {
            const float vv = __half2float(vbase[(size_t)(t0 + i) * hd + d]);
#pragma unroll
            for (int g = 0; g < kAttnMaxGroup; ++g)
                if (g < group) o[g] = fmaf(sc[g][i], vv, o[g]);
        }
        const int nchunks = gridDim.y;
#pragma unroll
        for (int g = 0; g < kAttnMaxGroup; ++g)
            if (g < group) part_o[((size_t)(kh * group + g) * nchunks + chunk) * hd + d] = o[g];
    }
    if (t < group) {
        const int nchunks = gridDim.y;
        part_ml[((size_t)(kh * group + t) * nchunks + chunk) * 2 + 0] = ml[t][0];
        part_ml[((size_t)(kh * group + t) * nchunks + chunk) * 2 + 1] = ml[t][1];
    }
}

// out[h][d] = sum_c o_c[d] e^{m_c - M} / sum_c l_c e^{m_c - M}, chunks in order.
__global__ void __launch_bounds__(256) attn_combine_kernel(const float* part_ml, const float* part_o, const int* pos_dev,
                                                           int nq, int hd, int max_ctx, int nchunks_alloc, float* out) {
    const int h = blockIdx.x;
    const int len = min(*pos_dev + 1, max_ctx);
    const int nchunks = (len + kAttnChunk - 1) / kAttnChunk;
    const float* ml = part_ml + (size_t)h * nchunks_alloc * 2;
    float M = -INFINITY;
    for (int c = 0; c < nchunks; ++c) M = fmaxf(M, ml[2 * c]);
    float L = 0.f;
    for (int c = 0; c < nchunks; ++c) L += ml[2 * c + 1] * expf(ml[2 * c] - M);
    for (int d = threadIdx.x; d < hd; d += blockDim.x) {
        float o = 0.f;
        for (int c = 0; c < nchunks; ++c) o = fmaf(part_o[((size_t)h * nchunks_alloc + c) * hd + d], expf(ml[2 * c] - M), o);
        out[(size_t)h * hd + d] = o / L;
    }
}

// ----------------------------------------------------------- SiLU-GLU ----

// out[i] = silu(gu[i]) * gu[n + i], silu(v) = v * sigmoid(v) with the sigmoid
// as 0.5 (tanh(v / 2) + 1) (recipe.rs:22662-22668).
__global__ void __launch_bounds__(256) silu_mul_kernel(const float* gu, int n, float* out) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        const float g = gu[i];
        out[i] = g * (0.5f * (tanhf(0.5f * g) + 1.0f)) * gu[n + i];
    }
}

// ------------------------------------------------------------- argmax ----

// The index of the largest value (the lowest index on a tie); one workgroup.
__global__ void __launch_bounds__(1024) argmax_kernel(const float* v, int n, int* out) {
    __shared__ float bv[1024];
    __shared__ int bi[1024];
    const int t = threadIdx.x;
    float best = -INFINITY;
    int idx = 0x7fffffff;
    for (int i = t; i < n; i += blockDim.x)
        if (v[i] > best) {  // ascending i: keeps the lowest index on a tie
            best = v[i];
            idx = i;
        }
    bv[t] = best;
    bi[t] = idx;
    __syncthreads();
    for (int s = blockDim.x / 2; s > 0; s >>= 1) {
        if (t < s) {
            const float ov = bv[t + s];
            const int oi = bi[t + s];
            if (ov > bv[t] || (ov == bv[t] && oi < bi[t])) {
                bv[t] = ov;
                bi[t] = oi;
            }
        }
        __syncthreads();
    }
    if (t == 0) *out = bi[0];
}

// out = table[token mod rows] (the next token's embedding row).
__global__ void __launch_bounds__(256) embed_row_kernel(const float* table, int rows, int n, const int* token,
                                                        float* out) {
    const int r = ((*token % rows) + rows) % rows;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
        out[i] = table[(size_t)r * n + i];
}

// Advances the decode position by one (the last launch of a captured step).
__global__ void advance_kernel(int* pos) {
    if (threadIdx.x == 0) *pos += 1;
}

// ------------------------------------------------------------ launches ----

hipError_t launch_add_rmsnorm(float* x, const float* delta, const float* w, int n, float eps, float* out,
                              hipStream_t stream) {
    hipLaunchKernelGGL(add_rmsnorm_kernel, dim3(1), dim3(1024), 0, stream, x, delta, w, n, eps, out);
    return hipGetLastError();
}

hipError_t launch_rope_kv(float* qkv, const int* pos, int nq, int nkv, int hd, double base, __half* kc, __half* vc,
                          int max_ctx, hipStream_t stream) {
    const int pairs = (nq + nkv) * (hd / 2);
    int grid = (pairs + 255) / 256;
    hipLaunchKernelGGL(rope_kv_kernel, dim3(grid), dim3(256), 0, stream, qkv, pos, nq, nkv, hd, base, kc, vc, max_ctx);
    return hipGetLastError();
}

size_t attention_workspace_bytes(int nq, int hd, int max_ctx) {
    const size_t nchunks = (size_t)(max_ctx + kAttnChunk - 1) / kAttnChunk;
    return nq * nchunks * 2 * sizeof(float) + nq * nchunks * (size_t)hd * sizeof(float);
}

hipError_t launch_attention(const float* q, const __half* kc, const __half* vc, const int* pos, int nq, int nkv,
                            int hd, int max_ctx, void* workspace, float* out, hipStream_t stream) {
    if (nkv < 1 || nq % nkv != 0 || nq / nkv > kAttnMaxGroup || hd % 64 != 0 || hd > kAttnMaxHead)
        return hipErrorInvalidValue;
    const int nchunks = (max_ctx + kAttnChunk - 1) / kAttnChunk;
    float* part_ml = static_cast<float*>(workspace);
    float* part_o = part_ml + (size_t)nq * nchunks * 2;
    const float scale = 1.0f / sqrtf((float)hd);
    // every chunk of the allocation runs; chunks past the position write -inf
    // maxima and zero sums that the combine ignores (it reads only the live ones)
    hipLaunchKernelGGL(attn_partial_kernel, dim3(nkv, nchunks), dim3(256), 0, stream, q, kc, vc, pos, nq, nkv, hd,
                       max_ctx, scale, part_ml, part_o);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(attn_combine_kernel, dim3(nq), dim3(256), 0, stream, part_ml, part_o, pos, nq, hd, max_ctx, nchunks,
                       out);
    return hipGetLastError();
}

hipError_t launch_silu_mul(const float* gu, int n, float* out, hipStream_t stream) {
    int grid = (n + 255) / 256;
    if (grid > 2048) grid = 2048;
    hipLaunchKernelGGL(silu_mul_kernel, dim3(grid), dim3(256), 0, stream, gu, n, out);
    return hipGetLastError();
}

hipError_t launch_argmax(const float* v, int n, int* out, hipStream_t stream) {
    hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(1024), 0, stream, v, n, out);
    return hipGetLastError();
}

hipError_t launch_embed_row(const float* table, int rows, int n, const int* token, float* out, hipStream_t stream) {
    int grid = (n + 255) / 256;
    if (grid > 256) grid = 256;
    hipLaunchKernelGGL(embed_row_kernel, dim3(grid), dim3(256), 0, stream, table, rows, n, token, out);
    return hipGetLastError();
}

hipError_t launch_advance(int* pos, hipStream_t stream) {
    hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(64), 0, stream, pos);
    return hipGetLastError();
}

}  // namespace rq
