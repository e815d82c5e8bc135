// recipe's int(8) sum on gfx950: the default precision profile's `sum = "int8"`
// with a 32-input step and the llama.cpp profile's 256-input step.
//
// The activation column of each position is rounded, in the workgroup's LDS,
// to Q8 records: per `step` inputs one fp32 step d and a signed byte per input
// (amd-nv-cpu.ll:1304-1500). Weight codes come from the repacked layout
// (layout.h) and dot the record bytes in v_dot4_i32_i8; every integer is exact,
// so the integer work is free to take any order, and the fp32 tail runs in
// recipe's order so each output carries recipe's bits.
//
// Reference: contraction_forward_gemv_wave_body on a backend with int8 dots
// (amd-nv-cpu.ll:1231-2241) and its slice helpers (build.rs:743-915).
// recipe's GPU backends run 32 lanes per output (NVIDIA warps, gfx11/gfx12
// wave32). Here each wave64 runs two outputs on its two 32-lane halves: lane l
// of a half holds exactly the partial sums recipe's lane l holds, and
// __shfl_xor within the half repeats recipe's butterfly.
//
// fp32 order per output (this file is built with -ffp-contract=off, and fmaf
// stands where recipe's state madd is):
//   16-value slices (Q4_K and Q6_K at a 32 step; Q8_0 and Q4_0 at either step):
//     lane l adds slices l, l+32, ... from +0; the lanes meet at offsets 16..1.
//       Q4_K  d8 * ((d*sc)*dot - (dmin*m)*sum)
//       Q6_K  d * (d8 * (sc * (dot - 32 sum)))
//       Q8_0, Q4_0  d8 * ((d*dot) + 0*sum), Q4_0's dot less 8 sum
//   Q4_K at a 256 step: acc = fma(dot_b, d*d8, acc), accmin = fma(min_b, dmin*d8,
//     accmin) per block in order (per quarter of the block for positions before
//     the last M % 4, unless the tail rule makes the last position whole); the
//     output is acc - accmin.
//   Q6_K at a 256 step: eight chains f_l = fma(d8*d, i_l, f_l) per block, added
//     as ((f0 + f4) + (f2 + f6)) + ((f1 + f5) + (f3 + f7)).
#include <hip/hip_runtime.h>

#include "chunk.h"
#include "kernels.h"

namespace rq {

namespace {

constexpr int kI8Threads = 256;                    // four waves, eight 32-lane halves
constexpr int kI8Halves = kI8Threads / 32;
constexpr int kI8RowsPerHalf = 2;                  // outputs each half takes per workgroup
constexpr int kI8Rows = kI8Halves * kI8RowsPerHalf;  // outputs per workgroup

// The Q8 records of one activation column of K inputs: d[K/32] and codes[K].
// Half-wave h takes steps h, h+halves, ...; lane v scans input v of each of
// the step's 32-value blocks, keeping the first extreme, and the halves'
// butterfly prefers the larger signed value between equal magnitudes
// (amd-nv-cpu.ll:1408-1470). inverse = -127 / extreme, d = 1 / inverse,
// code = clamp(round-half-even(x * inverse), -128, 127); an all-zero step
// has d = 0 and zero codes (amd-nv-cpu.ll:1447-1500).
__device__ __forceinline__ void q8_records(const float* __restrict__ x, int K, int step, float* d, int8_t* codes,
                                           int tid, int nthreads) {
    const int half = tid >> 5, lane = tid & 31, halves = nthreads >> 5;
    const int blocks = K >> 5, span = step >> 5;
    const int groups = (blocks + span - 1) / span;
    for (int g = half; g < groups; g += halves) {
        const int b0 = g * span, b1 = min(b0 + span, blocks);
        float e = 0.f;
        for (int b = b0; b < b1; ++b) {
            const float v = x[b * 32 + lane];
            if (fabsf(v) > fabsf(e)) e = v;
        }
#pragma unroll
        for (int off = 16; off > 0; off >>= 1) {
            const float p = __shfl_xor(e, off, 32);
            const float ap = fabsf(p), ae = fabsf(e);
            if (ap > ae || (ap == ae && p > e)) e = p;
        }
        const bool nonzero = fabsf(e) > 0.f;
        const float inverse_raw = -127.f / (nonzero ? e : 1.f);
        const float d_raw = 1.f / inverse_raw;
        const float inverse = nonzero ? inverse_raw : 0.f;
        const float dd = nonzero ? d_raw : 0.f;
        for (int b = b0; b < b1; ++b) {
            const float r = __builtin_rintf(x[b * 32 + lane] * inverse);
            codes[b * 32 + lane] = (int8_t)(int)fminf(fmaxf(r, -128.f), 127.f);
            if (lane == 0) d[b] = dd;
        }
    }
}

// Four consecutive 4-bit fields of word n (its low half, or its high half when
// `hi`) as four bytes, field k in byte k.
__device__ __forceinline__ uint32_t spread(uint32_t n, bool hi) {
    const uint32_t a = n & 0x0F0F0F0Fu, b = (n >> 4) & 0x0F0F0F0Fu;
    return __builtin_amdgcn_perm(b, a, hi ? 0x07030602u : 0x05010400u);
}
// Four stored nibbles (XOR 8, layout.h) as the codes q = nibble ^ 8, one per byte.
__device__ __forceinline__ uint32_t nib_codes(uint32_t n, bool hi) { return spread(n, hi) ^ 0x08080808u; }

__device__ __forceinline__ float f16_at(const uint8_t* p) {
    return (float)*reinterpret_cast<const _Float16*>(p);
}

// The int parts of one 16-value slice: dot = sum q*c over the slice (q the
// weight codes, c the record bytes), sum = sum c.
struct SliceInts {
    int dot, sum;
};

__device__ __forceinline__ int code_sum(const uint4& c) {
    int s = sdot4(0x01010101u, c.x, 0);
    s = sdot4(0x01010101u, c.y, s);
    s = sdot4(0x01010101u, c.z, s);
    return sdot4(0x01010101u, c.w, s);
}

__device__ __forceinline__ int dot4w(uint32_t q0, uint32_t q1, uint32_t q2, uint32_t q3, const uint4& c) {
    int s = sdot4(q0, c.x, 0);
    s = sdot4(q1, c.y, s);
    s = sdot4(q2, c.z, s);
    return sdot4(q3, c.w, s);
}

// Q4_K slice s of a row (block s/16, sub-block g = (s%16)/2, values 16*(s&1)..):
// its ints and the superblock's 16 meta bytes (d, dmin, packed scales).
__device__ __forceinline__ SliceInts q4k_slice(const uint8_t* rowp, int nch, int s, const uint4& c, uint4& meta) {
    const int b = s >> 4, l = s & 15, g = l >> 1;
    const ChunkPlace cp = chunk_place(Q4_K, b * 4 + (g >> 1), nch);
    const uint8_t* gs = rowp + cp.group_start;
    const uint2 n = *reinterpret_cast<const uint2*>(gs + ((g & 1) * cp.nb + cp.within) * 16 + (l & 1) * 8);
    meta = *reinterpret_cast<const uint4*>(gs + 2 * cp.nb * 16 + (cp.within >> 2) * 16);
    return SliceInts{dot4w(nib_codes(n.x, false), nib_codes(n.x, true), nib_codes(n.y, false), nib_codes(n.y, true), c),
                     code_sum(c)};
}

// get_scale_min_k4 of sub-block g from the superblock's meta words.
__device__ __forceinline__ void q4k_scale_min(const uint4& meta, int g, int& sc, int& m) {
    if (g < 4) {
        sc = (int)bfe(meta.y, 8 * g, 6);
        m = (int)bfe(meta.z, 8 * g, 6);
    } else {
        const int o = 8 * (g - 4);
        sc = (int)(bfe(meta.w, o, 4) | (bfe(meta.y, o + 6, 2) << 4));
        m = (int)(bfe(meta.w, o + 4, 4) | (bfe(meta.z, o + 6, 2) << 4));
    }
}

// Q6_K slice s (block s/16, scale group l = s%16): its ints, scale and d.
__device__ __forceinline__ SliceInts q6k_slice(const uint8_t* rowp, int nch, int s, const uint4& c, int& sc, float& d,
                                               int* words = nullptr) {
    const int b = s >> 4, l = s & 15, g4 = l & 3;
    const ChunkPlace cp = chunk_place(Q6_K, b * 4 + (l >> 2), nch);
    const uint8_t* gs = rowp + cp.group_start;
    const uint2 n = *reinterpret_cast<const uint2*>(gs + ((g4 >> 1) * cp.nb + cp.within) * 16 + (g4 & 1) * 8);
    const uint32_t H = *reinterpret_cast<const uint32_t*>(gs + (2 * cp.nb + cp.within) * 16 + g4 * 4);
    const uint8_t* meta = gs + 3 * cp.nb * 16;
    sc = (int)*reinterpret_cast<const int8_t*>(meta + (cp.within >> 2) * 16 + l);
    d = f16_at(meta + (cp.nb >> 2) * 16 + (cp.within >> 2) * 2);
    const uint32_t h0 = H & 0x33333333u, h1 = (H >> 2) & 0x33333333u;
    const uint32_t q0 = nib_codes(n.x, false) | (spread(h0, false) << 4);
    const uint32_t q1 = nib_codes(n.x, true) | (spread(h0, true) << 4);
    const uint32_t q2 = nib_codes(n.y, false) | (spread(h1, false) << 4);
    const uint32_t q3 = nib_codes(n.y, true) | (spread(h1, true) << 4);
    if (words) {
        words[0] = sdot4(q0, c.x, 0);
        words[1] = sdot4(q1, c.y, 0);
        words[2] = sdot4(q2, c.z, 0);
        words[3] = sdot4(q3, c.w, 0);
        return SliceInts{0, 0};
    }
    return SliceInts{dot4w(q0, q1, q2, q3, c), code_sum(c)};
}

// The fp32 value of slice s (build.rs:776-804, 845-848, 909-912).
template <int FMT>
__device__ __forceinline__ float slice_value(const uint8_t* rowp, int nch, int s, const int8_t* xc, const float* xd) {
    const uint4 c = *reinterpret_cast<const uint4*>(xc + s * 16);
    if constexpr (FMT == Q4_K) {
        uint4 meta;
        const SliceInts t = q4k_slice(rowp, nch, s, c, meta);
        int sc, m;
        const int g = (s & 15) >> 1;
        q4k_scale_min(meta, g, sc, m);
        const float group_d = half_lo(meta.x) * (float)sc;
        const float group_dmin = half_hi(meta.x) * (float)m;
        const float dot_scaled = group_d * (float)t.dot;
        const float minimum_scaled = group_dmin * (float)t.sum;
        const float value = dot_scaled - minimum_scaled;
        return xd[(s >> 4) * 8 + g] * value;
    } else if constexpr (FMT == Q6_K) {
        int sc;
        float d;
        const SliceInts t = q6k_slice(rowp, nch, s, c, sc, d);
        const int dot_signed = t.dot - t.sum * 32;
        const float scaled = (float)sc * (float)dot_signed;
        const float value = xd[s >> 1] * scaled;  // record (s/16)*8 + (s%16)/2
        return d * value;
    } else {
        const int blk = s >> 1, h = s & 1;
        int dot;
        float d;
        if constexpr (FMT == Q8_0) {
            const ChunkPlace cp = chunk_place(Q8_0, blk, nch);
            const uint8_t* gs = rowp + cp.group_start;
            const uint4 w = *reinterpret_cast<const uint4*>(gs + (h * cp.nb + cp.within) * 16);
            d = f16_at(gs + 2 * cp.nb * 16 + cp.within * 2);
            dot = dot4w(w.x, w.y, w.z, w.w, c);
        } else {
            const ChunkPlace cp = chunk_place(Q4_0, blk >> 1, nch);
            const uint8_t* gs = rowp + cp.group_start;
            const int part = blk & 1;
            const uint2 n = *reinterpret_cast<const uint2*>(gs + (part * cp.nb + cp.within) * 16 + h * 8);
            d = f16_at(gs + 2 * cp.nb * 16 + cp.within * 4 + part * 2);
            dot = dot4w(nib_codes(n.x, false), nib_codes(n.x, true), nib_codes(n.y, false), nib_codes(n.y, true), c);
        }
        const int sum = code_sum(c);
        if constexpr (FMT == Q4_0) dot -= sum * 8;
        const float minimum = 0.f;
        const float dot_scaled = d * (float)dot;
        const float minimum_scaled = minimum * (float)sum;
        const float value = dot_scaled + minimum_scaled;
        return xd[blk] * value;
    }
}

struct I8Launch {
    const uint8_t* w;
    int64_t row_bytes;
    int nch;
    int64_t rows;
    int K;
    const float* x;
    int64_t ldx;
    float* y;
    int64_t ldy;
    int M;
    int step;
    int tail;
};

__device__ __forceinline__ void stage_records(const I8Launch& p, int step, int8_t*& xc, float*& xd) {
    extern __shared__ __align__(16) uint8_t i8_lds[];
    xc = reinterpret_cast<int8_t*>(i8_lds);
    xd = reinterpret_cast<float*>(i8_lds + p.K);
    q8_records(p.x + (int64_t)blockIdx.y * p.ldx, p.K, step, xd, xc, (int)threadIdx.x, kI8Threads);
    __syncthreads();
}

// 16-value slices: lane l adds slices l, l+32, ...; the half's butterfly.
template <int FMT>
__global__ __launch_bounds__(kI8Threads) void int8_slices_kernel(I8Launch p) {
    int8_t* xc;
    float* xd;
    stage_records(p, p.step, xc, xd);
    const int half = (int)threadIdx.x >> 5, lane = (int)threadIdx.x & 31;
    const int slices = p.K >> 4;
    for (int i = 0; i < kI8RowsPerHalf; ++i) {
        const int64_t row = (int64_t)blockIdx.x * kI8Rows + i * kI8Halves + half;
        if (row >= p.rows) break;
        const uint8_t* rowp = p.w + row * p.row_bytes;
        float acc = 0.f;
        for (int s = lane; s < slices; s += 32) acc = acc + slice_value<FMT>(rowp, p.nch, s, xc, xd);
#pragma unroll
        for (int off = 16; off > 0; off >>= 1) acc = acc + __shfl_xor(acc, off, 32);
        if (lane == 0) p.y[(int64_t)blockIdx.y * p.ldy + row] = acc;
    }
}

// Q4_K at a 256 step (amd-nv-cpu.ll:1545-1733): lanes 0-15 of a half take the
// sixteen slices of one block and lanes 16-31 those of the next.
__global__ __launch_bounds__(kI8Threads) void int8_q4k256_kernel(I8Launch p) {
    int8_t* xc;
    float* xd;
    stage_records(p, 256, xc, xd);
    const int half = (int)threadIdx.x >> 5, lane = (int)threadIdx.x & 31, l = lane & 15, side = lane >> 4;
    const int m = (int)blockIdx.y;
    const bool whole = m >= p.M - (p.M & 3) || (p.tail && m == p.M - 1);
    const int nblk = p.K >> 8;
    for (int i = 0; i < kI8RowsPerHalf; ++i) {
        const int64_t row = (int64_t)blockIdx.x * kI8Rows + i * kI8Halves + half;
        if (row >= p.rows) break;
        const uint8_t* rowp = p.w + row * p.row_bytes;
        float acc = 0.f, accmin = 0.f;
        for (int b0 = 0; b0 < nblk; b0 += 2) {
            const int b = b0 + side;
            int di = 0, mi = 0;
            float scale = 0.f, dscale = 0.f;
            if (b < nblk) {
                const int s = b * 16 + l;
                uint4 meta;
                const SliceInts t = q4k_slice(rowp, p.nch, s, *reinterpret_cast<const uint4*>(xc + s * 16), meta);
                int sc, mn;
                q4k_scale_min(meta, l >> 1, sc, mn);
                di = sc * t.dot;
                mi = mn * t.sum;
                const float d8 = xd[b * 8];
                scale = half_lo(meta.x) * d8;
                dscale = half_hi(meta.x) * d8;
            }
            // Quarter sums (four slices each, exact) at lanes 4q of each side.
            di += __shfl_xor(di, 1, 32);
            mi += __shfl_xor(mi, 1, 32);
            di += __shfl_xor(di, 2, 32);
            mi += __shfl_xor(mi, 2, 32);
            const float s0 = __shfl(scale, 0, 32), ds0 = __shfl(dscale, 0, 32);
            const float s1 = __shfl(scale, 16, 32), ds1 = __shfl(dscale, 16, 32);
            if (whole) {
                di += __shfl_xor(di, 4, 32);
                mi += __shfl_xor(mi, 4, 32);
                di += __shfl_xor(di, 8, 32);
                mi += __shfl_xor(mi, 8, 32);
                acc = fmaf((float)__shfl(di, 0, 32), s0, acc);
                accmin = fmaf((float)__shfl(mi, 0, 32), ds0, accmin);
                if (b0 + 1 < nblk) {
                    acc = fmaf((float)__shfl(di, 16, 32), s1, acc);
                    accmin = fmaf((float)__shfl(mi, 16, 32), ds1, accmin);
                }
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    acc = fmaf((float)__shfl(di, 4 * q, 32), s0, acc);
                    accmin = fmaf((float)__shfl(mi, 4 * q, 32), ds0, accmin);
                }
                if (b0 + 1 < nblk) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        acc = fmaf((float)__shfl(di, 16 + 4 * q, 32), s1, acc);
                        accmin = fmaf((float)__shfl(mi, 16 + 4 * q, 32), ds1, accmin);
                    }
                }
            }
        }
        if (lane == 0) p.y[(int64_t)m * p.ldy + row] = acc - accmin;
    }
}

// Q6_K at a 256 step (amd-nv-cpu.ll:1836-2031, build.rs:871-884): lanes 0-15
// of a half take the slices of one block, 16-31 the next. Chain c takes word
// c%4 of the slices with parity c/4 (the four-value words at 4c of every
// 32-value group) and -32 times the scaled code sums of group c.
__global__ __launch_bounds__(kI8Threads) void int8_q6k256_kernel(I8Launch p) {
    int8_t* xc;
    float* xd;
    stage_records(p, 256, xc, xd);
    const int half = (int)threadIdx.x >> 5, lane = (int)threadIdx.x & 31, l = lane & 15, side = lane >> 4;
    const int chain = l & 7;
    const int nblk = p.K >> 8;
    for (int i = 0; i < kI8RowsPerHalf; ++i) {
        const int64_t row = (int64_t)blockIdx.x * kI8Rows + i * kI8Halves + half;
        if (row >= p.rows) break;
        const uint8_t* rowp = p.w + row * p.row_bytes;
        float f = 0.f;  // chain `chain`
        for (int b0 = 0; b0 < nblk; b0 += 2) {
            const int b = b0 + side;
            int W[4] = {0, 0, 0, 0}, G = 0;
            float scale = 0.f;
            if (b < nblk) {
                const int s = b * 16 + l;
                const uint4 c = *reinterpret_cast<const uint4*>(xc + s * 16);
                int sc, words[4];
                float d;
                q6k_slice(rowp, p.nch, s, c, sc, d, words);
#pragma unroll
                for (int k = 0; k < 4; ++k) W[k] = sc * words[k];
                G = -32 * (sc * code_sum(c));
                scale = xd[b * 8] * d;
            }
#pragma unroll
            for (int off = 2; off < 16; off <<= 1)
#pragma unroll
                for (int k = 0; k < 4; ++k) W[k] += __shfl_xor(W[k], off, 32);
            G += __shfl_xor(G, 1, 32);
            const int srcw = (lane & 16) + (chain >> 2);
            const int w0 = __shfl(W[0], srcw, 32), w1 = __shfl(W[1], srcw, 32);
            const int w2 = __shfl(W[2], srcw, 32), w3 = __shfl(W[3], srcw, 32);
            const int k = chain & 3;
            const int wpart = k == 0 ? w0 : (k == 1 ? w1 : (k == 2 ? w2 : w3));
            const int ic = wpart + __shfl(G, (lane & 16) + 2 * chain, 32);
            const int i0 = __shfl(ic, chain, 32), i1 = __shfl(ic, 16 + chain, 32);
            f = fmaf(__shfl(scale, 0, 32), (float)i0, f);
            if (b0 + 1 < nblk) f = fmaf(__shfl(scale, 16, 32), (float)i1, f);
        }
        const float t = f + __shfl_xor(f, 4, 32);
        const float u = t + __shfl_xor(t, 2, 32);
        const float total = u + __shfl_xor(u, 1, 32);
        if (lane == 0) p.y[(int64_t)blockIdx.y * p.ldy + row] = total;
    }
}

__global__ __launch_bounds__(kI8Threads) void q8_records_kernel(const float* x, int K, int step, float* d,
                                                                int8_t* codes) {
    q8_records(x, K, step, d, codes, (int)threadIdx.x, kI8Threads);
}

}  // namespace

size_t int8_lds_bytes(int64_t cols) { return (size_t)cols + (size_t)(cols / 32) * 4; }

hipError_t launch_matvec_int8(int fmt, const Planes& P, int64_t rows, int K, const float* x, int M, int64_t ldx,
                              float* y, int64_t ldy, int step, int tail, hipStream_t stream) {
    I8Launch p{P.base, P.row_bytes, P.nch, rows, K, x, ldx, y, ldy, M, step, tail};
    const dim3 grid((unsigned)((rows + kI8Rows - 1) / kI8Rows), (unsigned)M);
    const size_t lds = int8_lds_bytes(K);
    const bool blocks256 = step == 256 && (fmt == Q4_K || fmt == Q6_K);
    if (blocks256 && fmt == Q4_K)
        hipLaunchKernelGGL(int8_q4k256_kernel, grid, dim3(kI8Threads), lds, stream, p);
    else if (blocks256)
        hipLaunchKernelGGL(int8_q6k256_kernel, grid, dim3(kI8Threads), lds, stream, p);
    else if (fmt == Q4_K)
        hipLaunchKernelGGL(int8_slices_kernel<Q4_K>, grid, dim3(kI8Threads), lds, stream, p);
    else if (fmt == Q6_K)
        hipLaunchKernelGGL(int8_slices_kernel<Q6_K>, grid, dim3(kI8Threads), lds, stream, p);
    else if (fmt == Q8_0)
        hipLaunchKernelGGL(int8_slices_kernel<Q8_0>, grid, dim3(kI8Threads), lds, stream, p);
    else if (fmt == Q4_0)
        hipLaunchKernelGGL(int8_slices_kernel<Q4_0>, grid, dim3(kI8Threads), lds, stream, p);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_q8_records(const float* x, int K, int step, float* d, int8_t* codes, hipStream_t stream) {
    hipLaunchKernelGGL(q8_records_kernel, dim3(1), dim3(kI8Threads), 0, stream, x, K, step, d, codes);
    return hipGetLastError();
}

}  // namespace rq
