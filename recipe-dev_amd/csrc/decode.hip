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

#include <type_traits>

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

// Split over positions (flash decoding), in two launches.
//
// attention_kernel: one workgroup of kAttnThreads per (kv head, chunk of
// attn_chunk(HD) positions); a chunk is read once for every query head of its
// group. Lanes take one 16-byte piece (eight values) of a position's key and
// value: HD / 8 lanes per position, the whole chunk's keys and values loaded
// into registers before any arithmetic (addresses clamped into the cache;
// positions past the end are masked by selection, never by multiplying, so
// stale cache contents cannot leak in). Pass 1: each query head's score
// against each position (an eight-value dot per lane, summed over the
// position's lanes), times 1/sqrt(HD), kept in the registers of the
// position's lanes. Pass 2, per wave: each head's maximum mw over the wave's
// positions, weights e = exp(s - mw) and their sum lw, through DPP and lane
// swaps (no LDS, no barrier). Pass 3: o = sum e v, per lane over its
// positions, summed over the lanes that hold the same values; after the one
// barrier the waves are merged, m = max mw and each wave's o and lw scaled by
// e^(mw - m). The chunk's (m, l, o) go to the workspace.
//
// ROPE (the decode step's fused form): q and the new key come unrotated in
// qkv ([q heads | k heads | v heads]) and are turned here with a cos/sin table
// (rope_table_kernel); the chunk holding the position takes the new key and
// value (rounded to fp16, as the cache holds them) instead of the cache's
// entry and stores them into the cache.
//
// attn_combine_kernel: one workgroup per query head merges the live chunks,
// out = sum_c o_c e^(m_c - M) / sum_c l_c e^(m_c - M), chunks in order. Its
// loads do not depend on the position (every allocated chunk's partials are
// read and the dead ones dropped by selection), so they all go out at once.
//
// (A single launch whose last workgroup merges costs more: publishing the
// partial results across the XCDs' L2 caches takes an L2 write-back per
// workgroup.)
// Positions per chunk: 64, or 80 at head width 128 (five sweeps of 16
// positions), so that a context of 4,097 positions over 8 kv heads takes 416
// workgroups, at most two per CU, where 64 gave 520 and a third workgroup on
// one CU of every XCD.
__host__ __device__ constexpr int attn_chunk(int hd) { return hd == 128 ? 80 : 64; }
constexpr int kAttnThreads = 256;
constexpr int kAttnWaves = kAttnThreads / 64;
constexpr int kAttnMaxGroup = 8;      // query heads per kv head
constexpr int kAttnMaxChunks = 1024;  // max_ctx up to 65536

template <int LPP>
__device__ __forceinline__ float sum_lanes(float v) {
    // sum over aligned groups of LPP lanes (8, 16 or 32); every lane of a group gets the sum
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xf, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xf, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xf, 0xf, false));
    if constexpr (LPP >= 16)
        v += __builtin_bit_cast(float,
                                __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xf, 0xf, false));
    if constexpr (LPP >= 32) {  // lane ^ 16 through v_permlane16_swap (see swap16 below)
        float a = v, b = v;
        asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
        v = a + b;
    }
    return v;
}

// v combined with the value of lane ^ 16 and of lane ^ 32 through gfx950's
// VALU lane swaps (no LDS crossbar): v_permlane16_swap_b32 / 32 exchange odd
// 16-lane rows (upper 32 lanes) of the first register with even rows (lower
// 32 lanes) of the second; applied to two copies of v they leave, in every
// lane, the lower lane's value in the first and the upper lane's in the
// second. Written as inline assembly: this compiler's builtin loses the second
// result. The s_nop gives the wait states a VALU write needs before the swap
// reads it.
struct LanePair {
    float lo, hi;
};
__device__ __forceinline__ LanePair swap16(float v) {
    float a = v, b = v;
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
    return LanePair{a, b};
}
__device__ __forceinline__ LanePair swap32(float v) {
    float a = v, b = v;
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
    return LanePair{a, b};
}
__device__ __forceinline__ float swap16_sum(float v) {
    const LanePair p = swap16(v);
    return p.lo + p.hi;
}
__device__ __forceinline__ float swap32_sum(float v) {
    const LanePair p = swap32(v);
    return p.lo + p.hi;
}
__device__ __forceinline__ float swap16_max(float v) {
    const LanePair p = swap16(v);
    return fmaxf(p.lo, p.hi);
}
__device__ __forceinline__ float swap32_max(float v) {
    const LanePair p = swap32(v);
    return fmaxf(p.lo, p.hi);
}

// Maximum and sum over the 64 lanes of a wave, every lane getting the result:
// DPP within rows of 16, then the two lane swaps.
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xf, 0xf, false)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xf, 0xf, false)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xf, 0xf, false)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xf, 0xf, false)));
    return swap32_max(swap16_max(v));
}
__device__ __forceinline__ float wave_sum(float v) { return swap32_sum(swap16_sum(sum_lanes<16>(v))); }

// Maximum and sum over a wave's position slots: the lanes holding the same
// piece b of different positions (LPP lanes per position: lane bits from
// log2(LPP) up), every lane getting the result; DPP row rotation by 8 for
// lane bit 3, the lane swaps for bits 4 and 5.
template <int LPP>
__device__ __forceinline__ float slots_max(float v) {
    if constexpr (LPP <= 8)
        v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x128, 0xf, 0xf, false)));
    if constexpr (LPP <= 16) v = swap16_max(v);
    if constexpr (LPP <= 32) v = swap32_max(v);
    return v;
}
template <int LPP>
__device__ __forceinline__ float slots_sum(float v) {
    if constexpr (LPP <= 8)
        v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x128, 0xf, 0xf, false));
    if constexpr (LPP <= 16) v = swap16_sum(v);
    if constexpr (LPP <= 32) v = swap32_sum(v);
    return v;
}

struct AttnWork {
    float* ml;  // [nq][nchunks][2]
    float* o;   // [nq][nchunks][hd]
};

__host__ __device__ inline AttnWork attn_work(void* ws, int nq, int hd, int nchunks) {
    AttnWork w;
    w.ml = static_cast<float*>(ws);
    w.o = w.ml + (size_t)nq * nchunks * 2;
    return w;
}

__device__ __forceinline__ void load8(const float* p, float (&v)[8]) {
    const float4 a = *reinterpret_cast<const float4*>(p), c = *reinterpret_cast<const float4*>(p + 4);
    v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = c.x, v[5] = c.y, v[6] = c.z, v[7] = c.w;
}

__device__ __forceinline__ void unpack8(const uint4& r, float (&v)[8]) {
    const uint32_t w4[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int h2 = 0; h2 < 4; ++h2) {
        v[2 * h2] = half_lo(w4[h2]);
        v[2 * h2 + 1] = half_hi(w4[h2]);
    }
}

__device__ __forceinline__ uint4 pack8(const float (&v)[8]) {
    uint32_t w[4];
#pragma unroll
    for (int h2 = 0; h2 < 4; ++h2)
        w[h2] = (uint32_t)__half_as_ushort(__float2half(v[2 * h2])) |
                ((uint32_t)__half_as_ushort(__float2half(v[2 * h2 + 1])) << 16);
    return make_uint4(w[0], w[1], w[2], w[3]);
}

// NeoX rotation of the eight values x (dims 8b..8b+7 of a head, `upper` when
// they lie in the second half) given their partners xp (dims 8b +- HD/2) and
// the eight (cos, sin) pairs of pairs 8b mod HD/2 .. +7 at the position.
__device__ __forceinline__ void rotate8(float (&x)[8], const float (&xp)[8], const float2 (&cs)[8], bool upper) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        // lower half: x_i c - x_{i+half} s; upper half: x_{i+half} c + x_i s
        x[e] = upper ? x[e] * cs[e].x + xp[e] * cs[e].y : x[e] * cs[e].x - xp[e] * cs[e].y;
    }
}

// The rotation partners of a lane's eight values: in the lane holding the
// piece HD/2 away in the same position, lane ^ (LPP / 2). For 16 lanes per
// position that is a DPP rotation of each 16-lane row by 8, for 32 a 16-lane
// swap, for 8 a row shift by 4 (no LDS round trip in any case).
template <int LPP>
__device__ __forceinline__ void partners8(const float (&x)[8], float (&xp)[8]) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        if constexpr (LPP == 16) {
            xp[e] = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x[e]), 0x128, 0xf,
                                                                          0xf, false));  // row_ror:8
        } else if constexpr (LPP == 32) {
            const LanePair pr = swap16(x[e]);
            xp[e] = (threadIdx.x & 16) ? pr.lo : pr.hi;
        } else {  // 8 lanes per position: lane ^ 4, a row shift by 4 one way or the other
            const int iv = __builtin_bit_cast(int, x[e]);
            const int up = __builtin_amdgcn_update_dpp(0, iv, 0x114, 0xf, 0xf, false);    // row_shr:4 (lane - 4)
            const int down = __builtin_amdgcn_update_dpp(0, iv, 0x104, 0xf, 0xf, false);  // row_shl:4 (lane + 4)
            xp[e] = __builtin_bit_cast(float, (threadIdx.x & 4) ? up : down);
        }
    }
}

template <int HD, int MAXG, bool ROPE>
__global__ void __launch_bounds__(kAttnThreads) attention_kernel(const float* q, const float* kv_new, __half* kc,
                                                                 __half* vc, const float2* rope, const int* pos_dev,
                                                                 int nkv, int group, int max_ctx, float scale,
                                                                 AttnWork ws, int nchunks) {
    constexpr int LPP = HD / 8;                    // lanes per position
    constexpr int PPS = kAttnThreads / LPP;        // positions per sweep
    constexpr int CH = attn_chunk(HD);            // positions per chunk
    constexpr int NS = CH / PPS;                   // sweeps per chunk
    constexpr int HALF = HD / 2;
    __shared__ float wml[kAttnWaves][MAXG][2];  // each wave's (maximum, weight sum) per head
    // the partial outputs: with at most four query heads, one padded row per
    // position slot of the workgroup; with more, one row per wave
    constexpr bool kSlotRows = MAXG <= 4;
    constexpr int kRedRows = kSlotRows ? kAttnThreads / (HD / 8) : kAttnWaves;
    constexpr int kRedStride = MAXG * HD + (kSlotRows ? 4 : 0);
    __shared__ __align__(16) float red[kRedRows * kRedStride];
    const int kh = blockIdx.x, chunk = blockIdx.y;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int b = t % LPP, slot = t / LPP;
    const int t0 = chunk * CH;
    // Every load is issued before the first wait. The queries and, under ROPE,
    // the new key and value do not depend on the position, so they go out
    // while it is read; slots past the group read the group's last head (their
    // results are never written).
    float qr[MAXG][8];
#pragma unroll
    for (int g = 0; g < MAXG; ++g) load8(q + (size_t)(kh * group + min(g, group - 1)) * HD + b * 8, qr[g]);
    float kn[8], vn[8];
    if constexpr (ROPE) {
        load8(kv_new + (size_t)kh * HD + b * 8, kn);
        load8(kv_new + (size_t)(nkv + kh) * HD + b * 8, vn);
    }
    const int pos = *pos_dev;
    const int len = min(pos + 1, max_ctx);  // positions past the cache are not read
    if (t0 >= len) return;  // a chunk past the position: nothing to read (the whole workgroup leaves)

    // The position's (cos, sin) pairs for this lane's dims (the table has
    // max_ctx rows), requested before the keys and values: the rotation then
    // waits for them alone, and the scores for the keys alone.
    const bool upper = 8 * b >= HALF;
    float4 cs4v[ROPE ? 4 : 1];
    if constexpr (ROPE) {
        const float4* cs4 =
            reinterpret_cast<const float4*>(rope + (size_t)min(pos, max_ctx - 1) * HALF + (8 * b - (upper ? HALF : 0)));
#pragma unroll
        for (int i = 0; i < 4; ++i) cs4v[i] = cs4[i];
    }
    // keys and values of this lane's positions (clamped into the cache; masked below)
    uint4 kr[NS], vr[NS];
    // ROPE: the new position's key and value, rounded to fp16, stand in for
    // sweep jsel's cache entry where they are used (so that no wait for the
    // cache loads comes before the rotation)
    uint4 k16 = make_uint4(0, 0, 0, 0), v16 = make_uint4(0, 0, 0, 0);
    int jsel = -1;
    const size_t head_base = (size_t)kh * max_ctx;
#pragma unroll
    for (int j = 0; j < NS; ++j) {
        const int p = min(t0 + slot + j * PPS, max_ctx - 1);
        kr[j] = *reinterpret_cast<const uint4*>(kc + (head_base + p) * HD + b * 8);
    }
#pragma unroll
    for (int j = 0; j < NS; ++j) {
        const int p = min(t0 + slot + j * PPS, max_ctx - 1);
        vr[j] = *reinterpret_cast<const uint4*>(vc + (head_base + p) * HD + b * 8);
    }
    if constexpr (ROPE) {
        float2 cs[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 v = cs4v[i];
            cs[2 * i] = make_float2(v.x, v.y);
            cs[2 * i + 1] = make_float2(v.z, v.w);
        }
#pragma unroll
        for (int g = 0; g < MAXG; ++g) {
            float qp[8];
            partners8<LPP>(qr[g], qp);
            rotate8(qr[g], qp, cs, upper);
        }
        float kp[8];
        partners8<LPP>(kn, kp);
        rotate8(kn, kp, cs, upper);
        // the new position's key and value replace the cache entry in the chunk that holds it
        const int jn = pos - t0 - slot;
        k16 = pack8(kn);
        v16 = pack8(vn);
        if (pos < max_ctx && jn >= 0 && jn < CH && jn % PPS == 0) {
            *reinterpret_cast<uint4*>(kc + (head_base + pos) * HD + b * 8) = k16;
            *reinterpret_cast<uint4*>(vc + (head_base + pos) * HD + b * 8) = v16;
            jsel = jn / PPS;  // (the sweep whose key and value this lane takes from k16, v16)
        }
    }
    // The passes, in two forms: a chunk wholly before the new position (every
    // position live, none replaced by the new key and value) needs none of the
    // selections that mask dead positions or substitute the new entry; the
    // chunk holding the position, or past the cache's end, takes them. The
    // results are the same either way.
    float s[NS][MAXG], mw[MAXG], lw[MAXG], o[MAXG][8];
    auto passes = [&](auto full_tag) {
        constexpr bool FULL = decltype(full_tag)::value;
        // pass 1: each lane's positions' scores (every lane of a position holds them)
#pragma unroll
        for (int j = 0; j < NS; ++j) {
            float kv[8];
            unpack8(!FULL && j == jsel ? k16 : kr[j], kv);
            const bool live = FULL || t0 + slot + j * PPS < len;
#pragma unroll
            for (int g = 0; g < MAXG; ++g) {
                float d = 0.f;
#pragma unroll
                for (int e = 0; e < 8; ++e) d = fmaf(qr[g][e], kv[e], d);
                d = sum_lanes<LPP>(d);
                s[j][g] = live ? d * scale : -INFINITY;
            }
        }

        // pass 2, per wave: each head's maximum mw over the wave's positions (the
        // lane's sweeps, then the wave's position slots across lanes), weights
        // e = exp(s - mw) and their sum lw, all in registers; the chunk's waves
        // are merged at the end
#pragma unroll
        for (int g = 0; g < MAXG; ++g) {
            float m = s[0][g];
#pragma unroll
            for (int j = 1; j < NS; ++j) m = fmaxf(m, s[j][g]);
            mw[g] = slots_max<LPP>(m);
            float l = 0.f;
#pragma unroll
            for (int j = 0; j < NS; ++j) {
                s[j][g] = !FULL && s[j][g] == -INFINITY ? 0.f : __expf(s[j][g] - mw[g]);
                l += s[j][g];
            }
            lw[g] = slots_sum<LPP>(l);
        }

        // pass 3: o = sum_p e_p v_p over this lane's positions, then over the lanes
        // holding the same eight values (across the wave, then across waves)
#pragma unroll
        for (int g = 0; g < MAXG; ++g)
#pragma unroll
            for (int e = 0; e < 8; ++e) o[g][e] = 0.f;
#pragma unroll
        for (int j = 0; j < NS; ++j) {
            float vv[8];
            unpack8(!FULL && j == jsel ? v16 : vr[j], vv);
            if constexpr (!FULL) {
                const bool live = t0 + slot + j * PPS < len;
#pragma unroll
                for (int e = 0; e < 8; ++e) vv[e] = live ? vv[e] : 0.f;
            }
#pragma unroll
            for (int g = 0; g < MAXG; ++g)
#pragma unroll
                for (int e = 0; e < 8; ++e) o[g][e] = fmaf(s[j][g], vv[e], o[g][e]);
        }
    };
    // (wholly inside the live length and, under ROPE, wholly before the new
    // position)
    if (t0 + CH <= (ROPE ? min(pos, len) : len)) passes(std::true_type{});
    else passes(std::false_type{});
    if constexpr (kSlotRows) {
        // every lane's sums go to its slot's row; each output then adds the
        // rows in slot order (fewer instructions than lane exchanges)
        float* row = red + slot * kRedStride + b * 8;
#pragma unroll
        for (int g = 0; g < MAXG; ++g) {
            *reinterpret_cast<float4*>(row + g * HD) = make_float4(o[g][0], o[g][1], o[g][2], o[g][3]);
            *reinterpret_cast<float4*>(row + g * HD + 4) = make_float4(o[g][4], o[g][5], o[g][6], o[g][7]);
        }
    } else {
#pragma unroll
        for (int g = 0; g < MAXG; ++g)
#pragma unroll
            for (int e = 0; e < 8; ++e) o[g][e] = slots_sum<LPP>(o[g][e]);
        if (lane < LPP) {
            float* row = red + wave * kRedStride + b * 8;
#pragma unroll
            for (int g = 0; g < MAXG; ++g) {
                *reinterpret_cast<float4*>(row + g * HD) = make_float4(o[g][0], o[g][1], o[g][2], o[g][3]);
                *reinterpret_cast<float4*>(row + g * HD + 4) = make_float4(o[g][4], o[g][5], o[g][6], o[g][7]);
            }
        }
    }
    if (lane == 0) {
#pragma unroll
        for (int g = 0; g < MAXG; ++g) {
            wml[wave][g][0] = mw[g];
            wml[wave][g][1] = lw[g];
        }
    }
    __syncthreads();
    // the chunk: m = max over the waves, each wave's sums rescaled by e^(mw - m)
    constexpr int kRowsPerWave = kRedRows / kAttnWaves;
    for (int i = t; i < group * HD; i += kAttnThreads) {
        const int g = i / HD, d = i % HD;
        float m = wml[0][g][0];
#pragma unroll
        for (int w = 1; w < kAttnWaves; ++w) m = fmaxf(m, wml[w][g][0]);
        float acc = 0.f;
#pragma unroll
        for (int w = 0; w < kAttnWaves; ++w) {
            const float mwg = wml[w][g][0];
            const float f = mwg == -INFINITY ? 0.f : __expf(mwg - m);
            float part = 0.f;
#pragma unroll
            for (int r = 0; r < kRowsPerWave; ++r) part += red[(w * kRowsPerWave + r) * kRedStride + i];
            acc = fmaf(f, part, acc);
        }
        ws.o[((size_t)(kh * group + g) * nchunks + chunk) * HD + d] = acc;
    }
    if (t < group) {
        float m = wml[0][t][0];
#pragma unroll
        for (int w = 1; w < kAttnWaves; ++w) m = fmaxf(m, wml[w][t][0]);
        float l = 0.f;
#pragma unroll
        for (int w = 0; w < kAttnWaves; ++w) {
            const float mwg = wml[w][t][0];
            l = fmaf(mwg == -INFINITY ? 0.f : __expf(mwg - m), wml[w][t][1], l);
        }
        ws.ml[((size_t)(kh * group + t) * nchunks + chunk) * 2 + 0] = m;
        ws.ml[((size_t)(kh * group + t) * nchunks + chunk) * 2 + 1] = l;
    }
}

// out[h] = sum_c w_c o_c with w_c = e^(m_c - M) / sum_c l_c e^(m_c - M) over
// the live chunks of query head h. Each thread takes one 16-byte column of the
// head and every CLN-th chunk; its first kPre chunks' partials and maxima are
// loaded with the position, before anything is known of which are live. Each
// wave forms the maximum and weight sum of every 256th chunk's (m, l) from
// its lanes; after one barrier every thread merges the four waves' into M and
// L, weights its own chunks, and the chunk lanes are summed in order through
// LDS.
template <int HD>
__global__ void __launch_bounds__(256) attn_combine_kernel(AttnWork ws, const int* pos_dev, int max_ctx, int nchunks,
                                                           float* out) {
    constexpr int COLS4 = HD / 4;
    constexpr int CLN = 256 / COLS4;
    constexpr int kPre = 12;
    constexpr int kMlPer = kAttnMaxChunks / 256;
    __shared__ float part[2][4];
    __shared__ float4 cred[256];
    const int h = blockIdx.x, t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const float* hml = ws.ml + (size_t)h * nchunks * 2;
    const int col = t % COLS4, cl = t / COLS4;
    const float* po = ws.o + (size_t)h * nchunks * HD + col * 4;
    float4 pre[kPre];
    float mine[kPre];  // the maxima of the thread's own chunks
#pragma unroll
    for (int k = 0; k < kPre; ++k) {
        const int c = min(cl + k * CLN, nchunks - 1);
        pre[k] = *reinterpret_cast<const float4*>(po + (size_t)c * HD);
        mine[k] = hml[2 * c];
    }
    float2 mlv[kMlPer];
#pragma unroll
    for (int k = 0; k < kMlPer; ++k) {
        const int c = min(t + 256 * k, nchunks - 1);
        mlv[k] = *reinterpret_cast<const float2*>(hml + 2 * c);
    }
    const int len = min(*pos_dev + 1, max_ctx);
    const int live = (len + attn_chunk(HD) - 1) / attn_chunk(HD);
    // this wave's maximum and weight sum over its lanes' live chunks
    float Mw = -INFINITY;
#pragma unroll
    for (int k = 0; k < kMlPer; ++k)
        if (t + 256 * k < live) Mw = fmaxf(Mw, mlv[k].x);
    Mw = wave_max(Mw);  // (DPP and lane swaps: no LDS round trips)
    float Lw = 0.f;
#pragma unroll
    for (int k = 0; k < kMlPer; ++k)
        if (t + 256 * k < live) Lw = fmaf(mlv[k].y, __expf(mlv[k].x - Mw), Lw);
    Lw = wave_sum(Lw);
    if (lane == 0) {
        part[0][wave] = Mw;
        part[1][wave] = Lw;
    }
    __syncthreads();
    const float M = fmaxf(fmaxf(part[0][0], part[0][1]), fmaxf(part[0][2], part[0][3]));
    float L = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w)
        if (part[0][w] != -INFINITY) L = fmaf(part[1][w], __expf(part[0][w] - M), L);
    const float inv = 1.0f / L;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int k = 0; k < kPre; ++k) {
        const int c = cl + k * CLN;
        if (c < live) {
            const float w = __expf(mine[k] - M);
            acc.x = fmaf(w, pre[k].x, acc.x);
            acc.y = fmaf(w, pre[k].y, acc.y);
            acc.z = fmaf(w, pre[k].z, acc.z);
            acc.w = fmaf(w, pre[k].w, acc.w);
        }
    }
    for (int c = cl + kPre * CLN; c < live; c += CLN) {
        const float4 v = *reinterpret_cast<const float4*>(po + (size_t)c * HD);
        const float w = __expf(hml[2 * c] - M);
        acc.x = fmaf(w, v.x, acc.x);
        acc.y = fmaf(w, v.y, acc.y);
        acc.z = fmaf(w, v.z, acc.z);
        acc.w = fmaf(w, v.w, acc.w);
    }
    cred[t] = acc;
    __syncthreads();
    if (t < COLS4) {
        float4 o4 = cred[t];
        for (int k = 1; k < CLN; ++k) {
            const float4 v = cred[k * COLS4 + t];
            o4.x += v.x, o4.y += v.y, o4.z += v.z, o4.w += v.w;
        }
        o4.x *= inv, o4.y *= inv, o4.z *= inv, o4.w *= inv;
        *reinterpret_cast<float4*>(out + (size_t)h * HD + t * 4) = o4;
    }
}

// table[p][i] = (cos, sin) of p * base^(-2i/head_dim), the angle and its cosine
// and sine in f64 (as rope_kv_kernel takes them), rounded to fp32.
__global__ void __launch_bounds__(256) rope_table_kernel(float2* table, int half, int head_dim, double base, int rows) {
    const double lb = log(base);
    for (int u = blockIdx.x * 256 + threadIdx.x; u < rows * half; u += gridDim.x * 256) {
        const int p = u / half, i = u % half;
        const double angle = (double)p * exp(-((double)(2 * i) / (double)head_dim) * lb);
        table[u] = make_float2((float)cos(angle), (float)sin(angle));
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

// The index of the largest value (the lowest index on a tie; NaNs are
// skipped), in two launches: kArgmaxBlocks workgroups each take a contiguous
// slice and leave their best (value, index) in the workspace, then one
// workgroup reduces those.
constexpr int kArgmaxBlocks = 128;
constexpr int kArgmaxThreads = 256;

__device__ __forceinline__ bool beats(float v, int i, float bv, int bi) {
    return v > bv || (v == bv && i < bi);
}

__device__ __forceinline__ void block_best(float& best, int& idx) {
    __shared__ float bv[kArgmaxThreads];
    __shared__ int bi[kArgmaxThreads];
    const int t = threadIdx.x;
    bv[t] = best;
    bi[t] = idx;
    __syncthreads();
    for (int s = kArgmaxThreads / 2; s > 0; s >>= 1) {
        if (t < s && beats(bv[t + s], bi[t + s], bv[t], bi[t])) {
            bv[t] = bv[t + s];
            bi[t] = bi[t + s];
        }
        __syncthreads();
    }
    best = bv[0];
    idx = bi[0];
}

__global__ void __launch_bounds__(kArgmaxThreads) argmax_part_kernel(const float* v, int n, float* part_v,
                                                                     int* part_i) {
    const int t = threadIdx.x;
    const int per = (n + gridDim.x - 1) / gridDim.x;
    const int lo = blockIdx.x * per, hi = min(n, lo + per);
    float best = -INFINITY;
    int idx = 0x7fffffff;
    for (int i = lo + t; i < hi; i += kArgmaxThreads) {
        const float x = v[i];
        if (beats(x, i, best, idx)) {
            best = x;
            idx = i;
        }
    }
    block_best(best, idx);
    if (t == 0) {
        part_v[blockIdx.x] = best;
        part_i[blockIdx.x] = idx;
    }
}

__global__ void __launch_bounds__(kArgmaxThreads) argmax_final_kernel(const float* part_v, const int* part_i, int parts,
                                                                      int* out) {
    const int t = threadIdx.x;
    float best = -INFINITY;
    int idx = 0x7fffffff;
    for (int b = t; b < parts; b += kArgmaxThreads)
        if (beats(part_v[b], part_i[b], best, idx)) {
            best = part_v[b];
            idx = part_i[b];
        }
    block_best(best, idx);
    if (t == 0) *out = idx == 0x7fffffff ? 0 : idx;
}

// out = table[token mod rows] (the next token's embedding row).
__global__ void __launch_bounds__(256) embed_row_kernel(const float* table, int rows, int n, const int* token,
                                                        float* out) {
    const int r = ((*token % rows) + rows) % rows;
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) out[i] = table[(size_t)r * n + i];
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
    const size_t nchunks = (size_t)(max_ctx + attn_chunk(hd) - 1) / attn_chunk(hd);
    return (nq * nchunks * 2 + nq * nchunks * (size_t)hd) * sizeof(float);
}

struct AttnLaunch {
    const float* q;
    const float* kv_new;
    __half* kc;
    __half* vc;
    const float2* rope;
    const int* pos;
    int nkv, group, max_ctx, nchunks;
    AttnWork ws;
    float* out;
};

template <int HD, int MAXG, bool ROPE>
static void launch_attention_t(const AttnLaunch& a, hipStream_t stream) {
    const float scale = 1.0f / sqrtf((float)HD);
    hipLaunchKernelGGL((attention_kernel<HD, MAXG, ROPE>), dim3(a.nkv, a.nchunks), dim3(kAttnThreads), 0, stream, a.q,
                       a.kv_new, a.kc, a.vc, a.rope, a.pos, a.nkv, a.group, a.max_ctx, scale, a.ws, a.nchunks);
    hipLaunchKernelGGL((attn_combine_kernel<HD>), dim3(a.nkv * a.group), dim3(256), 0, stream, a.ws, a.pos, a.max_ctx,
                       a.nchunks, a.out);
}

template <int HD, bool ROPE>
static void launch_attention_hd(const AttnLaunch& a, hipStream_t stream) {
    if (a.group <= 1)
        launch_attention_t<HD, 1, ROPE>(a, stream);
    else if (a.group <= 2)
        launch_attention_t<HD, 2, ROPE>(a, stream);
    else if (a.group <= 4)
        launch_attention_t<HD, 4, ROPE>(a, stream);
    else
        launch_attention_t<HD, 8, ROPE>(a, stream);
}

template <bool ROPE>
static hipError_t launch_attention_any(int hd, const AttnLaunch& a, hipStream_t stream) {
    // every chunk of the allocation is launched (the grid stays fixed while the
    // position advances under a captured graph); chunks past the position leave at once
    if (hd == 64)
        launch_attention_hd<64, ROPE>(a, stream);
    else if (hd == 128)
        launch_attention_hd<128, ROPE>(a, stream);
    else
        launch_attention_hd<256, ROPE>(a, stream);
    return hipGetLastError();
}

static bool attention_shape_ok(int nq, int nkv, int hd, int max_ctx) {
    return nkv >= 1 && nq % nkv == 0 && nq / nkv <= kAttnMaxGroup && (hd == 64 || hd == 128 || hd == 256) &&
           max_ctx <= kAttnMaxChunks * attn_chunk(hd);
}

hipError_t launch_attention(const float* q, const __half* kc, const __half* vc, const int* pos, int nq, int nkv,
                            int hd, int max_ctx, void* workspace, float* out, hipStream_t stream) {
    if (!attention_shape_ok(nq, nkv, hd, max_ctx)) return hipErrorInvalidValue;
    AttnLaunch a;
    a.q = q;
    a.kv_new = nullptr;
    a.kc = const_cast<__half*>(kc);  // read only without ROPE
    a.vc = const_cast<__half*>(vc);
    a.rope = nullptr;
    a.pos = pos;
    a.nkv = nkv;
    a.group = nq / nkv;
    a.max_ctx = max_ctx;
    a.nchunks = (max_ctx + attn_chunk(hd) - 1) / attn_chunk(hd);
    a.ws = attn_work(workspace, nq, hd, a.nchunks);
    a.out = out;
    return launch_attention_any<false>(hd, a, stream);
}

hipError_t launch_attention_rope(const float* qkv, const float2* rope_table, __half* kc, __half* vc, const int* pos,
                                 int nq, int nkv, int hd, int max_ctx, void* workspace, float* out,
                                 hipStream_t stream) {
    if (!attention_shape_ok(nq, nkv, hd, max_ctx)) return hipErrorInvalidValue;
    AttnLaunch a;
    a.q = qkv;
    a.kv_new = qkv + (size_t)nq * hd;
    a.kc = kc;
    a.vc = vc;
    a.rope = rope_table;
    a.pos = pos;
    a.nkv = nkv;
    a.group = nq / nkv;
    a.max_ctx = max_ctx;
    a.nchunks = (max_ctx + attn_chunk(hd) - 1) / attn_chunk(hd);
    a.ws = attn_work(workspace, nq, hd, a.nchunks);
    a.out = out;
    return launch_attention_any<true>(hd, a, stream);
}

hipError_t launch_rope_table(float2* table, int head_dim, double base, int rows, hipStream_t stream) {
    const int half = head_dim / 2;
    int grid = (rows * half + 255) / 256;
    if (grid > 4096) grid = 4096;
    hipLaunchKernelGGL(rope_table_kernel, dim3(grid), dim3(256), 0, stream, table, half, head_dim, base, rows);
    return hipGetLastError();
}

hipError_t launch_silu_mul(const float* gu, int n, float* out, hipStream_t stream) {
    int grid = (n + 255) / 256;
    if (grid > 2048) grid = 2048;
    hipLaunchKernelGGL(silu_mul_kernel, dim3(grid), dim3(256), 0, stream, gu, n, out);
    return hipGetLastError();
}

size_t argmax_workspace_bytes() { return kArgmaxBlocks * (sizeof(float) + sizeof(int)); }

hipError_t launch_argmax(const float* v, int n, int* out, void* workspace, hipStream_t stream) {
    float* part_v = static_cast<float*>(workspace);
    int* part_i = reinterpret_cast<int*>(part_v + kArgmaxBlocks);
    const int blocks = n < kArgmaxBlocks * kArgmaxThreads ? (n + kArgmaxThreads - 1) / kArgmaxThreads : kArgmaxBlocks;
    hipLaunchKernelGGL(argmax_part_kernel, dim3(blocks), dim3(kArgmaxThreads), 0, stream, v, n, part_v, part_i);
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(kArgmaxThreads), 0, stream, part_v, part_i, blocks, out);
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
