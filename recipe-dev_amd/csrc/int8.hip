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
// lane exchanges within the half (lane_xor) repeat recipe's butterfly.
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

constexpr int kI8Threads = 512;                  // eight waves
constexpr int kI8Rows = 2 * (kI8Threads / 64);   // outputs per workgroup: two per wave

// Extreme selection of recipe's Q8 records (amd-nv-cpu.ll:1422-1470): the
// partner replaces the running extreme when its magnitude is larger, or equal
// with a larger signed value. Scanning values in any order from +0 with this
// rule yields the value recipe's 32-lane butterfly leaves: the maximum under
// (magnitude, signed value), zeros and NaNs never replacing +0.
__device__ __forceinline__ bool extreme_wins(float p, float e) {
    const float ap = fabsf(p), ae = fabsf(e);
    return ap > ae || (ap == ae && p > e);
}

// inverse = -127 / extreme and d = 1 / inverse, both correctly rounded; an
// all-zero step has inverse 0 and d 0 (amd-nv-cpu.ll:1447-1456).
__device__ __forceinline__ void step_of(float e, float& inverse, float& d) {
    const bool nonzero = fabsf(e) > 0.f;
    const float inverse_raw = -127.f / (nonzero ? e : 1.f);
    const float d_raw = 1.f / inverse_raw;
    inverse = nonzero ? inverse_raw : 0.f;
    d = nonzero ? d_raw : 0.f;
}

// The 32 inputs of one record from a 16-byte aligned row.
__device__ __forceinline__ void load_record(const float* __restrict__ xr, float4 (&xv)[8]) {
#pragma unroll
    for (int q = 0; q < 8; ++q) xv[q] = reinterpret_cast<const float4*>(xr)[q];
}

// The 32 codes of a record in registers: clamp(round-half-even(x * inverse),
// -128, 127) (amd-nv-cpu.ll:1484-1490), written to LDS.
__device__ __forceinline__ void record_codes(const float4 (&xv)[8], float inverse, int8_t* out) {
    uint32_t w[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        const float f[4] = {xv[q].x, xv[q].y, xv[q].z, xv[q].w};
        uint32_t word = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float rr = __builtin_rintf(f[k] * inverse);
            word |= ((uint32_t)(int)fminf(fmaxf(rr, -128.f), 127.f) & 0xffu) << (8 * k);
        }
        w[q] = word;
    }
    reinterpret_cast<uint4*>(out)[0] = make_uint4(w[0], w[1], w[2], w[3]);
    reinterpret_cast<uint4*>(out)[1] = make_uint4(w[4], w[5], w[6], w[7]);
}

// Record r at a 32 step from its 32 inputs in registers: the extreme, the
// step d[r] and the codes.
__device__ __forceinline__ void record_from_registers(const float4 (&xv)[8], float* d, int8_t* codes, int r) {
    float e = 0.f;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        if (extreme_wins(xv[q].x, e)) e = xv[q].x;
        if (extreme_wins(xv[q].y, e)) e = xv[q].y;
        if (extreme_wins(xv[q].z, e)) e = xv[q].z;
        if (extreme_wins(xv[q].w, e)) e = xv[q].w;
    }
    float inverse, dd;
    step_of(e, inverse, dd);
    record_codes(xv, inverse, codes + r * 32);
    d[r] = dd;
}

// The Q8 records of one activation row of K inputs (16-byte aligned) into
// LDS: codes[K], d[K/32], and ginv[ceil(K/256)] scratch for a 256 step.
// Step 32: one thread per record scans its 32 inputs. Step 256: recipe's lane
// v keeps the first largest magnitude among input v of the step's 32-value
// blocks (amd-nv-cpu.ll:1408-1440), computed here by one thread per (step,
// lane) into `codes` (free until the codes are written); one thread per step
// then takes the extreme over its 32 lanes. Ends with a barrier.
__device__ __forceinline__ void q8_records(const float* __restrict__ x, int K, int step, float* d, int8_t* codes,
                                           float* ginv, int tid, int nthreads) {
    const int blocks = K >> 5;
    if (step == 32) {
        for (int r = tid; r < blocks; r += nthreads) {
            float4 xv[8];
            load_record(x + r * 32, xv);
            record_from_registers(xv, d, codes, r);
        }
        __syncthreads();
        return;
    }
    const int groups = (blocks + 7) >> 3;
    float* lane_best = reinterpret_cast<float*>(codes);  // groups * 32 floats <= K bytes
    for (int i = tid; i < groups * 32; i += nthreads) {
        const int g = i >> 5, v = i & 31;
        const int b1 = min(g * 8 + 8, blocks);
        float e = 0.f;
        for (int b = g * 8; b < b1; ++b) {
            const float xv = x[b * 32 + v];
            if (fabsf(xv) > fabsf(e)) e = xv;
        }
        lane_best[i] = e;
    }
    __syncthreads();
    for (int g = tid; g < groups; g += nthreads) {
        float e = 0.f;
        for (int v = 0; v < 32; ++v) {
            const float p = lane_best[g * 32 + v];
            if (extreme_wins(p, e)) e = p;
        }
        float inverse, dd;
        step_of(e, inverse, dd);
        ginv[g] = inverse;
        for (int b = g * 8; b < min(g * 8 + 8, blocks); ++b) d[b] = dd;
    }
    __syncthreads();
    for (int r = tid; r < blocks; r += nthreads) {
        float4 xv[8];
        load_record(x + r * 32, xv);
        record_codes(xv, ginv[r >> 3], codes + r * 32);
    }
    __syncthreads();
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

// get_scale_min_k4 of sub-block g from the superblock's meta words (the
// chunk fields of q4k_field).
__device__ __forceinline__ void q4k_scale_min(const uint4& meta, int g, int& sc, int& m) {
    const uint32_t f = q4k_field(meta, g >> 1);
    sc = (int)bfe(f, 12 * (g & 1), 6);
    m = (int)bfe(f, 12 * (g & 1) + 6, 6);
}

// The dot of 16 stored nibbles (two words, XOR 8) with a slice's record bytes.
__device__ __forceinline__ int q4_dot(uint32_t n0, uint32_t n1, const uint4& c) {
    return dot4w(nib_codes(n0, false), nib_codes(n0, true), nib_codes(n1, false), nib_codes(n1, true), c);
}

// Q6_K slice t (0..3) of a chunk: codes q = l | h << 4, four per word.
__device__ __forceinline__ void q6_words(const ChunkData<Q6_K>& D, int t, uint32_t q[4]) {
    const uint4& lo = D.q[t >> 1];
    const uint32_t n0 = (t & 1) ? lo.z : lo.x, n1 = (t & 1) ? lo.w : lo.y;
    const uint32_t H = word(D.q[2], t);
    const uint32_t h0 = H & 0x33333333u, h1 = (H >> 2) & 0x33333333u;
    q[0] = nib_codes(n0, false) | (spread(h0, false) << 4);
    q[1] = nib_codes(n0, true) | (spread(h0, true) << 4);
    q[2] = nib_codes(n1, false) | (spread(h1, false) << 4);
    q[3] = nib_codes(n1, true) | (spread(h1, true) << 4);
}

__device__ __forceinline__ uint4 record_bytes(const int8_t* xc, int s) {
    return *reinterpret_cast<const uint4*>(xc + s * 16);
}

// Slices per chunk: a chunk is 64 weights (four 16-value slices) except
// Q8_0's 32 (two).
template <int FMT>
constexpr int chunk_slices() {
    return FMT == Q8_0 ? 2 : 4;
}

// The fp32 values of chunk c's slices (build.rs:776-804, 845-848, 909-912),
// slice t of the chunk being slice c * chunk_slices + t of the row.
template <int FMT>
__device__ __forceinline__ void chunk_values(const ChunkData<FMT>& D, int c, const int8_t* xc, const float* xd,
                                             float v[chunk_slices<FMT>()]) {
    if constexpr (FMT == Q4_K) {
        const float d = half_lo(D.meta.x), dmin = half_hi(D.meta.x);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int s = 4 * c + t, j = t >> 1, h = t & 1;
            const int g = 2 * (c & 3) + j;
            const uint4 x = record_bytes(xc, s);
            int sc, m;
            q4k_scale_min(D.meta, g, sc, m);
            const float group_d = d * (float)sc;
            const float group_dmin = dmin * (float)m;
            const float dot_scaled = group_d * (float)q4_dot(word(D.q[j], 2 * h), word(D.q[j], 2 * h + 1), x);
            const float minimum_scaled = group_dmin * (float)code_sum(x);
            const float value = dot_scaled - minimum_scaled;
            v[t] = xd[(c >> 2) * 8 + g] * value;
        }
    } else if constexpr (FMT == Q6_K) {
        const float d = half_lo(D.meta.y);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int s = 4 * c + t;
            const uint4 x = record_bytes(xc, s);
            uint32_t q[4];
            q6_words(D, t, q);
            const int dot_signed = dot4w(q[0], q[1], q[2], q[3], x) - code_sum(x) * 32;
            const float scaled = (float)sbfe(D.meta.x, 8 * t, 8) * (float)dot_signed;
            const float value = xd[s >> 1] * scaled;
            v[t] = d * value;
        }
    } else if constexpr (FMT == Q8_0) {
        const float d = half_lo(D.meta.x);
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const uint4 x = record_bytes(xc, 2 * c + t);
            const uint4& w = D.q[t];
            const int sum = code_sum(x);
            const float minimum = 0.f;
            const float dot_scaled = d * (float)dot4w(w.x, w.y, w.z, w.w, x);
            const float minimum_scaled = minimum * (float)sum;
            const float value = dot_scaled + minimum_scaled;
            v[t] = xd[c] * value;
        }
    } else {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int s = 4 * c + t, j = t >> 1, h = t & 1;
            const uint4 x = record_bytes(xc, s);
            const float d = j ? half_hi(D.meta.x) : half_lo(D.meta.x);
            const int sum = code_sum(x);
            const int dot = q4_dot(word(D.q[j], 2 * h), word(D.q[j], 2 * h + 1), x) - sum * 8;
            const float minimum = 0.f;
            const float dot_scaled = d * (float)dot;
            const float minimum_scaled = minimum * (float)sum;
            const float value = dot_scaled + minimum_scaled;
            v[t] = xd[2 * c + j] * value;
        }
    }
}

struct I8Launch {
    Planes P;
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

// LDS: the records' codes (K bytes), steps (K/32 floats) and per-step
// inverses (ceil(K/256) floats), then per wave two rows of 256 slice values.
__device__ __forceinline__ void stage_records(const I8Launch& p, int step, int8_t*& xc, float*& xd, float*& rowbuf) {
    extern __shared__ __align__(16) uint8_t i8_lds[];
    xc = reinterpret_cast<int8_t*>(i8_lds);
    xd = reinterpret_cast<float*>(i8_lds + p.K);
    const int tail_floats = (p.K >> 5) + ((p.K + 255) >> 8);
    rowbuf = xd + ((tail_floats + 3) & ~3) + ((int)threadIdx.x >> 6) * 512;
    q8_records(p.x + (int64_t)blockIdx.y * p.ldx, p.K, step, xd, xc, xd + (p.K >> 5), (int)threadIdx.x, kI8Threads);
}

// Exact int sums over the four lanes of a quad (one 256-value block).
__device__ __forceinline__ int quad_sum(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xf, 0xf, false);  // lane ^ 1
    return v + __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xf, 0xf, false);  // lane ^ 2
}
__device__ __forceinline__ int lane_int(int v, int lane) { return __builtin_amdgcn_readlane(v, lane); }
// The value of lane ^ OFF (OFF < 32, within the lane's 32-lane half), through
// DPP and the 16-lane swap rather than the LDS crossbar: quad permutations
// for 1 and 2, row shifts by 4 either way for 4, a row rotation by 8 for 8,
// v_permlane16_swap for 16. Each lane then adds exactly the partner
// __shfl_xor would give it, so the butterflies keep their bits.
template <int OFF>
__device__ __forceinline__ float lane_xor(float v) {
    const int iv = __builtin_bit_cast(int, v);
    if constexpr (OFF == 1) return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, iv, 0xB1, 0xf, 0xf, false));
    if constexpr (OFF == 2) return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, iv, 0x4E, 0xf, 0xf, false));
    if constexpr (OFF == 4) {
        const int up = __builtin_amdgcn_update_dpp(0, iv, 0x114, 0xf, 0xf, false);    // row_shr:4 (lane - 4)
        const int down = __builtin_amdgcn_update_dpp(0, iv, 0x104, 0xf, 0xf, false);  // row_shl:4 (lane + 4)
        return __builtin_bit_cast(float, (threadIdx.x & 4) ? up : down);
    }
    if constexpr (OFF == 8) return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, iv, 0x128, 0xf, 0xf, false));
    if constexpr (OFF == 16) {
        float a = v, b = v;
        asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
        return (threadIdx.x & 16) ? a : b;
    }
    static_assert(OFF == 1 || OFF == 2 || OFF == 4 || OFF == 8 || OFF == 16, "lane_xor: 1, 2, 4, 8 or 16");
    return v;
}

__device__ __forceinline__ float lane_float(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// 16-value slices. Each wave takes two rows at a time, lane i decoding chunk
// i of each 64-chunk pass; the pass's slice values go to the wave's LDS rows,
// where recipe's lane l (lanes 0-31 for the first row, 32-63 for the second)
// adds slices l, l+32, ... in order; the halves' butterflies end each row.
template <int FMT>
__global__ __launch_bounds__(kI8Threads) void int8_slices_kernel(I8Launch p) {
    constexpr int CS = chunk_slices<FMT>();
    int8_t* xc;
    float* xd;
    float* rowbuf;
    const int tid = (int)threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int64_t row0 = (int64_t)blockIdx.x * kI8Rows + 2 * wave;
    const bool live = row0 < p.rows, two = row0 + 1 < p.rows;
    const int slices = p.K >> 4, nch = p.P.nch;
    // At a 32 step with at most one record per thread, the inputs of the
    // thread's record are loaded first and the first pass's weights after
    // them, so that waiting for the inputs leaves the weight loads in flight
    // (the counter of outstanding loads drains in order).
    const int blocks = p.K >> 5;
    const bool early = p.step == 32 && blocks <= kI8Threads;
    ChunkData<FMT> A, B;
    bool have = false;
    if (early) {
        extern __shared__ __align__(16) uint8_t i8_lds[];
        xc = reinterpret_cast<int8_t*>(i8_lds);
        xd = reinterpret_cast<float*>(i8_lds + p.K);
        const int tail_floats = (p.K >> 5) + ((p.K + 255) >> 8);
        rowbuf = xd + ((tail_floats + 3) & ~3) + wave * 512;
        float4 xv[8];
        if (tid < blocks) load_record(p.x + (int64_t)blockIdx.y * p.ldx + tid * 32, xv);
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("" ::: "memory");
        if (live && lane < nch) {
            load_chunk<FMT>(p.P, row0, lane, A);
            if (two) load_chunk<FMT>(p.P, row0 + 1, lane, B);
            have = true;
        }
        if (tid < blocks) record_from_registers(xv, xd, xc, tid);
        __syncthreads();
    } else {
        stage_records(p, p.step, xc, xd, rowbuf);
    }
    if (!live) return;
    const int mine = lane >> 5;  // which of the two rows this lane sums
    float acc = 0.f;
    for (int c0 = 0; c0 < nch; c0 += 64) {
        const int c = c0 + lane;
        if (c < nch && !(have && c0 == 0)) {
            load_chunk<FMT>(p.P, row0, c, A);
            if (two) load_chunk<FMT>(p.P, row0 + 1, c, B);
        }
        if (c < nch) {
            float va[CS], vb[CS] = {};
            chunk_values<FMT>(A, c, xc, xd, va);
            if (two) chunk_values<FMT>(B, c, xc, xd, vb);
#pragma unroll
            for (int t = 0; t < CS; ++t) {
                rowbuf[lane * CS + t] = va[t];
                rowbuf[256 + lane * CS + t] = vb[t];
            }
        }
        __builtin_amdgcn_wave_barrier();
        const int base = c0 * CS;  // first slice of the pass
        const float* mybuf = rowbuf + 256 * mine;
        const int l = lane & 31;
#pragma unroll
        for (int j = 0; j < 2 * CS; ++j) {
            const int s = base + l + 32 * j;
            if (s < slices) acc = acc + mybuf[l + 32 * j];
        }
        __builtin_amdgcn_wave_barrier();
    }
    acc = acc + lane_xor<16>(acc);
    acc = acc + lane_xor<8>(acc);
    acc = acc + lane_xor<4>(acc);
    acc = acc + lane_xor<2>(acc);
    acc = acc + lane_xor<1>(acc);
    if ((lane & 31) == 0 && (mine == 0 || two)) p.y[(int64_t)blockIdx.y * p.ldy + row0 + mine] = acc;
}

// Q4_K at a 256 step (amd-nv-cpu.ll:1545-1733). Lane i decodes chunk i of a
// pass: quarter i%4 of block i/4, whose two sub-blocks give the quarter's
// exact ints (scale times dot, minimum times code sum). Each pass leaves, per
// row and block, the four quarters' ints and the block's two scales in the
// wave's LDS row (ten words per block); lanes 0 and 1 (first row) and 32 and
// 33 (second row) then run the acc and accmin fma chains in block order.
__device__ __forceinline__ void q4k256_ints(const ChunkData<Q4_K>& D, int c, const int8_t* xc, const float* xd,
                                            float* out) {
    int dq = 0, mq = 0;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int g = 2 * (c & 3) + j;
        int sc, m;
        q4k_scale_min(D.meta, g, sc, m);
        const uint4 x0 = record_bytes(xc, 4 * c + 2 * j), x1 = record_bytes(xc, 4 * c + 2 * j + 1);
        dq += sc * (q4_dot(word(D.q[j], 0), word(D.q[j], 1), x0) + q4_dot(word(D.q[j], 2), word(D.q[j], 3), x1));
        mq += m * (code_sum(x0) + code_sum(x1));
    }
    float* blk = out + (c & 63) / 4 * 10;
    blk[2 * (c & 3)] = __builtin_bit_cast(float, dq);
    blk[2 * (c & 3) + 1] = __builtin_bit_cast(float, mq);
    if ((c & 3) == 0) {
        const float d8 = xd[(c >> 2) * 8];
        blk[8] = half_lo(D.meta.x) * d8;
        blk[9] = half_hi(D.meta.x) * d8;
    }
}

__global__ __launch_bounds__(kI8Threads) void int8_q4k256_kernel(I8Launch p) {
    int8_t* xc;
    float* xd;
    float* rowbuf;
    stage_records(p, 256, xc, xd, rowbuf);
    const int wave = (int)threadIdx.x >> 6, lane = (int)threadIdx.x & 63;
    const int64_t row0 = (int64_t)blockIdx.x * kI8Rows + 2 * wave;
    if (row0 >= p.rows) return;
    const bool two = row0 + 1 < p.rows;
    const int m = (int)blockIdx.y;
    const bool whole = m >= p.M - (p.M & 3) || (p.tail && m == p.M - 1);
    const int nch = p.P.nch;
    const int chain = lane & 1;                        // 0: acc, 1: accmin
    const float* mine = rowbuf + 256 * (lane >> 5);  // the row this lane's chain belongs to
    float acc = 0.f;
    for (int c0 = 0; c0 < nch; c0 += 64) {
        const int c = c0 + lane;
        ChunkData<Q4_K> A, B;
        if (c < nch) {
            load_chunk<Q4_K>(p.P, row0, c, A);
            if (two) load_chunk<Q4_K>(p.P, row0 + 1, c, B);
            q4k256_ints(A, c, xc, xd, rowbuf);
            if (two) q4k256_ints(B, c, xc, xd, rowbuf + 256);
        }
        __builtin_amdgcn_wave_barrier();
        if ((lane & 31) < 2) {
            const int blocks = min(16, (nch - c0) >> 2);
            for (int b = 0; b < blocks; ++b) {
                const float* blk = mine + b * 10;
                const float s = blk[8 + chain];
                if (whole) {
                    const int w = (__builtin_bit_cast(int, blk[chain]) + __builtin_bit_cast(int, blk[2 + chain])) +
                                  (__builtin_bit_cast(int, blk[4 + chain]) + __builtin_bit_cast(int, blk[6 + chain]));
                    acc = fmaf((float)w, s, acc);
                } else {
#pragma unroll
                    for (int q = 0; q < 4; ++q) acc = fmaf((float)__builtin_bit_cast(int, blk[2 * q + chain]), s, acc);
                }
            }
        }
        __builtin_amdgcn_wave_barrier();
    }
    const float other = lane_xor<1>(acc);
    if (lane == 0) p.y[(int64_t)m * p.ldy + row0] = acc - other;
    if (lane == 32 && two) p.y[(int64_t)m * p.ldy + row0 + 1] = acc - other;
}

// Q6_K at a 256 step (amd-nv-cpu.ll:1836-2031, build.rs:871-884). Lane i
// decodes chunk i of a pass: quarter i%4 of block i/4, slices 4(i%4)+t. Chain
// k takes word k%4 of the slices with parity k/4 (the four-value words at 4k
// of every 32-value group) and -32 times the scaled code sums of group k. The
// quads' exact sums give each block's eight chain ints, left with the block's
// scale in the wave's LDS row (nine words per block); lanes 0-7 (first row)
// and 32-39 (second row) each run one chain's fmas in block order.
__device__ __forceinline__ void q6k256_ints(const ChunkData<Q6_K>& D, int c, const int8_t* xc, const float* xd,
                                            float* out) {
    const int qq = c & 3;
    int I[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int G0 = 0, G1 = 0;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const uint4 x = record_bytes(xc, 4 * c + t);
        const int sc = sbfe(D.meta.x, 8 * t, 8);
        uint32_t q[4];
        q6_words(D, t, q);
        I[(t & 1) * 4 + 0] += sc * sdot4(q[0], x.x, 0);
        I[(t & 1) * 4 + 1] += sc * sdot4(q[1], x.y, 0);
        I[(t & 1) * 4 + 2] += sc * sdot4(q[2], x.z, 0);
        I[(t & 1) * 4 + 3] += sc * sdot4(q[3], x.w, 0);
        const int g = -32 * (sc * code_sum(x));
        if (t < 2)
            G0 += g;
        else
            G1 += g;
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        I[k] += (k == 2 * qq ? G0 : 0) + (k == 2 * qq + 1 ? G1 : 0);
        I[k] = quad_sum(I[k]);
    }
    if (qq == 0) {
        float* blk = out + (c & 63) / 4 * 9;
#pragma unroll
        for (int k = 0; k < 8; ++k) blk[k] = __builtin_bit_cast(float, I[k]);
        blk[8] = xd[(c >> 2) * 8] * half_lo(D.meta.y);
    }
}

__global__ __launch_bounds__(kI8Threads) void int8_q6k256_kernel(I8Launch p) {
    int8_t* xc;
    float* xd;
    float* rowbuf;
    stage_records(p, 256, xc, xd, rowbuf);
    const int wave = (int)threadIdx.x >> 6, lane = (int)threadIdx.x & 63;
    const int64_t row0 = (int64_t)blockIdx.x * kI8Rows + 2 * wave;
    if (row0 >= p.rows) return;
    const bool two = row0 + 1 < p.rows;
    const int nch = p.P.nch;
    const int chain = lane & 7;
    const float* mine = rowbuf + 256 * (lane >> 5);
    float f = 0.f;
    for (int c0 = 0; c0 < nch; c0 += 64) {
        const int c = c0 + lane;
        ChunkData<Q6_K> A, B;
        if (c < nch) {  // whole quads: nch is a multiple of four
            load_chunk<Q6_K>(p.P, row0, c, A);
            if (two) load_chunk<Q6_K>(p.P, row0 + 1, c, B);
            q6k256_ints(A, c, xc, xd, rowbuf);
            if (two) q6k256_ints(B, c, xc, xd, rowbuf + 256);
        }
        __builtin_amdgcn_wave_barrier();
        if ((lane & 31) < 8) {
            const int blocks = min(16, (nch - c0) >> 2);
            for (int b = 0; b < blocks; ++b) {
                const float* blk = mine + b * 9;
                f = fmaf(blk[8], (float)__builtin_bit_cast(int, blk[chain]), f);
            }
        }
        __builtin_amdgcn_wave_barrier();
    }
    const float t = f + lane_xor<4>(f);
    const float u = t + lane_xor<2>(t);
    const float total = u + lane_xor<1>(u);
    if (lane == 0) p.y[(int64_t)blockIdx.y * p.ldy + row0] = total;
    if (lane == 32 && two) p.y[(int64_t)blockIdx.y * p.ldy + row0 + 1] = total;
}

// The records of one row, staged as the products stage them, then copied out.
__global__ __launch_bounds__(kI8Threads) void q8_records_kernel(const float* x, int K, int step, float* d,
                                                                int8_t* codes) {
    extern __shared__ __align__(16) uint8_t i8_lds[];
    int8_t* xc = reinterpret_cast<int8_t*>(i8_lds);
    float* xd = reinterpret_cast<float*>(i8_lds + K);
    q8_records(x, K, step, xd, xc, xd + (K >> 5), (int)threadIdx.x, kI8Threads);
    for (int i = (int)threadIdx.x; i < K; i += kI8Threads) codes[i] = xc[i];
    for (int i = (int)threadIdx.x; i < (K >> 5); i += kI8Threads) d[i] = xd[i];
}

}  // namespace

// codes, steps, per-step inverses (rounded up to 16 bytes), then 2 KiB of
// slice values per wave.
size_t int8_lds_bytes(int64_t cols) {
    const size_t tail = (size_t)(cols / 32) + (size_t)((cols + 255) / 256);
    return (size_t)cols + ((tail + 3) & ~size_t(3)) * 4 + (size_t)(kI8Threads / 64) * 2048;
}

hipError_t launch_matvec_int8(int fmt, const Planes& P, int64_t rows, int K, const float* x, int M, int64_t ldx,
                              float* y, int64_t ldy, int step, int tail, hipStream_t stream) {
    I8Launch p{P, rows, K, x, ldx, y, ldy, M, step, tail};
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
    hipLaunchKernelGGL(q8_records_kernel, dim3(1), dim3(kI8Threads), int8_lds_bytes(K), stream, x, K, step, d, codes);
    return hipGetLastError();
}

}  // namespace rq
