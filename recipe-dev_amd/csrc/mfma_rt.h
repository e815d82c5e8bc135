// Small-M (3 <= M <= 32) quantized products on the matrix cores, fp16
// activations: the streaming form.
//
// Each wave owns a 16-row tile of W and a range of K. Weights are read in the
// repacked layout with 64-byte runs per row (RB = 16 rows x 4 chunks x 16
// bytes per load instruction) or 128-byte runs (RB = 8 rows x 8 chunks), and
// turned into the matrix core's B operand inside registers: a load leaves
// word j of chunk c of row r in lane (r, c); the B operand of a 32-weight
// block wants word kq of that block's row n in lane (n, kq). That is a
// transpose between lane bits and register indices, done with
// v_permlane16_swap / v_permlane32_swap (lane bits 4 and 5) and a DPP row
// rotation by 8 (lane bit 3): two or three exchanges per word, no LDS.
//
// Activations and block scales never pass through registers on their way to
// LDS: buffer_load ... lds writes a lane's 16 bytes at the instruction's LDS
// base + 16 lane, which is exactly the matrix core's A-operand order when
// lane (m, kq) loads x[m][32 b + 8 kq .. + 7] -- one load instruction per
// 1 KiB fragment. The scale table of the wave's rows over its K range is
// loaded the same way once, at the start. A step's activation tiles are
// shared by the waves of the workgroup (one barrier per step), in D + 1
// buffers: tiles for step s + D land while step s reads its own. The
// kernel waits for these loads itself (the compiler cannot tell the buffers
// apart and would otherwise wait for every load before any LDS read).
// Weight registers rotate through D + 1 sets with the loop unrolled D + 1
// times, so that no set is copied around the loop.
//
// A workgroup is WR row tiles x WK K ranges: tall matrices use WR = 4 (the
// activation window is shared by four tiles), mid-sized ones 4 x 2, shorter
// ones 2 x 2 or 1 x 4 (split K, the partial sums added in LDS in a fixed
// order at the end, so results are deterministic). Above 16 activation rows a
// wave takes two 16-row tiles, or (few row tiles) the launch takes one
// workgroup row per 16-row half.
//
// Each 32-weight block is one v_mfma_f32_16x16x32_f16 per 16 activation rows
// on exact fp16 weight codes, scaled into fp32 sums per block (Q4_K: minus its
// minimum times the block's activation sums, from a second product with a
// block of ones; Q6_K: a block spans two 16-weight scale groups, so a second
// product with the second group's weights zeroed gives the first group's sum,
// and the difference the second's). Products are exact; sums are fp32.
#pragma once

#include <hip/hip_ext.h>

#include <type_traits>

#include "halfcode.h"
#include "kernels.h"

namespace rq {

typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

template <int FMT> struct RtFmt;
// BPC: 32-weight blocks per chunk; QB: LDS bytes of one quad's scales (four
// chunks); DB: extra LDS bytes per quad (Q6_K's d, as fp32).
template <> struct RtFmt<Q4_0> { static constexpr int BPC = 2, QB = 16, DB = 0; };
template <> struct RtFmt<Q4_K> { static constexpr int BPC = 2, QB = 16, DB = 0; };
template <> struct RtFmt<Q8_0> { static constexpr int BPC = 1, QB = 8, DB = 0; };
template <> struct RtFmt<Q6_K> { static constexpr int BPC = 2, QB = 16, DB = 4; };

constexpr int kRtDepth = 2;       // steps of weights and activations in flight
constexpr int kRtMaxQuads = 48;   // quads (four chunks) of scales per wave and row, at most

template <int FMT, int RB, int NT, int WR, int WK>
struct RtCfg {
    static constexpr int CPS = 64 / RB;                       // chunks per step and row
    static constexpr int NI = 16 / RB;                        // load instructions per part and step
    static constexpr int QP = Traits<FMT>::QP;
    static constexpr int NB = CPS * RtFmt<FMT>::BPC;          // 32-weight blocks per step
    static constexpr int W = WR * WK;
    static constexpr int XWIN = NB * NT * 1024;               // one K range's activations for a step
    static constexpr int XBUF = WK * XWIN;                    // one step, every K range
    static constexpr int XI = NB * NT * WK / W;               // 1 KiB activation tiles each wave loads per step
    static constexpr int NXB = kRtDepth + 1;                  // activation buffers (a step's tiles land while
                                                              // the buffer is free: D steps ahead, one in use)
    // The scale table of a wave: 16 rows x `quads` quads, loaded straight
    // into LDS in whole load instructions (64 lanes x 16 bytes for 16-byte
    // quads, 64 x 4 bytes otherwise), then Q6_K's d per quad (64 x 4 bytes).
    static constexpr int QB = RtFmt<FMT>::QB;
    static constexpr int SPI = QB == 16 ? 1024 : 256;         // bytes one scale load instruction writes
    static constexpr int MS = (16 * kRtMaxQuads * QB + SPI - 1) / SPI;  // scale load instructions (the most)
    static constexpr int MD = FMT == Q6_K ? (16 * kRtMaxQuads * 4 + 255) / 256 : 0;
    static constexpr int s_bytes(int quads) { return (16 * quads * QB + SPI - 1) / SPI * SPI; }
    static constexpr int d_bytes(int quads) { return FMT == Q6_K ? (16 * quads * 4 + 255) / 256 * 256 : 0; }
    static constexpr int DUMMY = 1024;                        // where surplus scale loads write
    // LDS bytes of a launch whose waves cover `quads` quads each
    static constexpr int lds_bytes(int quads) { return NXB * XBUF + DUMMY + W * (s_bytes(quads) + d_bytes(quads)); }
    static_assert((NB * NT) % WR == 0, "activation items must divide over the workgroup");
};

// v_permlane16_swap / v_permlane32_swap exchange the off-diagonal halves of two
// registers across lane bit 4 / 5; a DPP row rotation by 8 does it for bit 3.
__device__ __forceinline__ void swap_bit4(uint32_t& a, uint32_t& b) {
    const auto r = __builtin_amdgcn_permlane16_swap(a, b, false, false);
    a = r[0];
    b = r[1];
}
__device__ __forceinline__ void swap_bit5(uint32_t& a, uint32_t& b) {
    const auto r = __builtin_amdgcn_permlane32_swap(a, b, false, false);
    a = r[0];
    b = r[1];
}
__device__ __forceinline__ void swap_bit3(uint32_t& a, uint32_t& b, bool hi) {
    const uint32_t ra = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)a, 0x128, 0xF, 0xF, false);  // row_ror:8
    const uint32_t rb = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)b, 0x128, 0xF, 0xF, false);
    a = hi ? rb : a;
    b = hi ? b : ra;
}

// R[h][j]: word j of a load instruction h's 16 bytes (lane = (row, chunk) as
// loaded). Afterwards T[c] = R[c & 1][c >> 1] (RB = 8) or R[0][c] (RB = 16)
// holds word kq of chunk c for lane (row n, kq).
template <int RB>
__device__ __forceinline__ void transpose_words(uint32_t (&R)[16 / RB][4], int lane) {
    if constexpr (RB == 8) {
        const bool hi = (lane & 8) != 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) swap_bit3(R[0][j], R[1][j], hi);
    }
#pragma unroll
    for (int h = 0; h < 16 / RB; ++h) {
        swap_bit4(R[h][0], R[h][1]);
        swap_bit4(R[h][2], R[h][3]);
        swap_bit5(R[h][0], R[h][2]);
        swap_bit5(R[h][1], R[h][3]);
    }
}

// 16 bytes per lane from a buffer straight into LDS at `lds_addr` + 16 lane
// (buffer_load_dwordx4 ... lds; M0 holds the LDS address). Written as inline
// assembly so that the compiler's wait placement does not treat every later
// LDS read as depending on it (it cannot tell the activation buffers apart):
// the kernel waits for these loads itself.
__device__ __forceinline__ void lds_load16(const u32x4_t& rsrc, uint32_t voffset, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
                 :
                 : "v"(voffset), "s"(rsrc), "s"(lds_addr)
                 : "memory", "m0");
}

// 4 bytes per lane, likewise (lane L's dword at `lds_addr` + 4 L).
__device__ __forceinline__ void lds_load4(const u32x4_t& rsrc, uint32_t voffset, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dword %0, %1, 0 offen lds"
                 :
                 : "v"(voffset), "s"(rsrc), "s"(lds_addr)
                 : "memory", "m0");
}

// nibbles_to_h with its mask and magic held in VGPRs (`mk` = 0x00F0000F,
// `mg` = 0x54006400): a VOP3 and-or takes two VGPR operands where gfx9 allows
// only one constant.
__device__ __forceinline__ void nibbles_to_h_v(uint32_t w, uint32_t neg, uint32_t mk, uint32_t mg, uint32_t (&o)[4]) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const uint32_t sel = (uint32_t)t | 0x0c00u | ((uint32_t)t << 16) | 0x0c000000u;
        const uint32_t b = __builtin_amdgcn_perm(0u, w, sel);
        o[t] = pk_add_h((b & mk) | mg, neg);
    }
}

template <int RB>
__device__ __forceinline__ uint32_t tword(const uint32_t (&R)[16 / RB][4], int c) {
    if constexpr (RB == 8) return R[c & 1][c >> 1];
    else return R[0][c];
}

// Launched on a grid of (row tile groups) x (activation row groups of 16 NT):
// workgroup row blockIdx.y takes activation rows [16 NT y, 16 NT y + 16 NT),
// so that a product at 32 rows can run as two 16-row halves (twice the waves,
// each decoding the weights for its half).
template <int FMT, int RB, int NT, int WR, int WK>
__global__ void __launch_bounds__(64 * WR * WK) __attribute__((amdgpu_waves_per_eu(2))) matvec_mfma_rt(MvParams p, int M, uint32_t x_bytes, int steps_per_wave) {
    using C = RtCfg<FMT, RB, NT, WR, WK>;
    using F = RtFmt<FMT>;
    constexpr int CPS = C::CPS, NI = C::NI, QP = C::QP, NB = C::NB, D = kRtDepth;
    extern __shared__ uint4 smem[];
    uint8_t* lds = reinterpret_cast<uint8_t*>(smem);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);  // (uniform: scalar arithmetic below)
    const int wr = wave % WR, wk = wave / WR;
    // this workgroup's activation rows (the host launches ceil(M / 16 NT) rows of workgroups)
    {
        const int m0 = 16 * NT * (int)blockIdx.y;
        const uint32_t skip = (uint32_t)((int64_t)m0 * p.ldx * 2);
        p.x = static_cast<const uint16_t*>(p.x) + (int64_t)m0 * p.ldx;
        p.y += (int64_t)m0 * p.ldy;
        x_bytes -= skip;
        M -= m0;
    }
    uint8_t* const xbase = lds;
    uint8_t* const dummy = lds + C::NXB * C::XBUF;
    const int nq_row = steps_per_wave * CPS / 4;  // quads per row of the LDS scale table
    const int wave_meta = C::s_bytes(nq_row) + C::d_bytes(nq_row);
    uint8_t* const meta = dummy + C::DUMMY + wave * wave_meta;  // scales [row][quad]
    uint8_t* const meta_d = meta + C::s_bytes(nq_row);                             // Q6_K: d [row][quad]

    const int64_t row0 = ((int64_t)blockIdx.x * WR + wr) * 16;
    const int nch = p.P.nch;
    const int total_steps = (nch + CPS - 1) / CPS;
    // this wave's steps: [s_begin, s_begin + steps_per_wave) of the K range wk
    const int s_begin = (int)(((int64_t)total_steps * wk) / WK);
    const int s_end = (int)(((int64_t)total_steps * (wk + 1)) / WK);
    const __amdgpu_buffer_rsrc_t rs = planes_rsrc(p.P);
    const __amdgpu_buffer_rsrc_t xrs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p.x), (short)0, (int)x_bytes, 0x00020000);
    const int ln = lane % RB, lc = lane / RB;   // loader: row within the instruction, chunk of the step
    const int mn = lane & 15, kq = lane >> 4;   // matrix core: row n / activation row m, k slice


    // ---- scales of the wave's rows over its K range ----
    const int q_begin = s_begin * CPS / 4;
    const int nq = (s_end - s_begin) * CPS / 4;  // quads of this range (<= nq_row <= kRtMaxQuads)
    const int total_quads = (nch + 3) / 4;
    const uint32_t gbytes = full_group_bytes<FMT>();
    // byte offset of the scale region of quad gq's group in row r: it follows
    // the group's QP code parts; QB bytes per quad, then Q6_K's fp16 d per quad
    auto region_of = [&](int r, int gq, int& nb) {
        const int group = gq >> 4;
        const int rest = nch - (group << 6);
        nb = rest > 64 ? 64 : rest;
        return (uint32_t)(row0 + r) * (uint32_t)p.P.row_bytes + (uint32_t)group * gbytes + (uint32_t)(QP * nb * 16);
    };
    // ---- weights and activations of a step ----
    // wbuf[slot][part][h][j]; the Q6_K high part is kept as its own part index
    typedef uint32_t WSet[QP][NI][4];
    // Per-lane parts of the load offsets, fixed for the whole loop; the step's
    // own parts are wave-uniform (a step's chunks lie inside one 64-chunk group).
    uint32_t wrow[NI];
    bool wrow_ok[NI];
#pragma unroll
    for (int h = 0; h < NI; ++h) {
        const int64_t row = row0 + RB * h + ln;
        wrow_ok[h] = row < p.rows;
        wrow[h] = (uint32_t)row * (uint32_t)p.P.row_bytes + (uint32_t)lc * 16u;
    }
    auto load_w = [&](int s, WSet& w) {
        const int c0 = s * CPS;
        const uint32_t group = (uint32_t)c0 >> 6;
        const uint32_t rest = (uint32_t)nch - (group << 6);
        const uint32_t nb = rest > 64u ? 64u : rest;
        const uint32_t gbase = group * gbytes + (((uint32_t)c0 & 63u) << 4);
        const bool step_ok = s < s_end && c0 < nch;
        const bool lane_ok = c0 + lc < nch;
#pragma unroll
        for (int h = 0; h < NI; ++h) {
            const uint32_t keep = step_ok && lane_ok && wrow_ok[h] ? 0xFFFFFFFFu : 0u;
#pragma unroll
            for (int part = 0; part < QP; ++part) {
                const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(
                    rs, oob_unless(wrow[h] + gbase + (uint32_t)part * nb * 16u, keep), 0, 0);
                w[part][h][0] = v[0];
                w[part][h][1] = v[1];
                w[part][h][2] = v[2];
                w[part][h][3] = v[3];
            }
        }
    };
    // Activation tile i of a step: the 1 KiB A fragment of tile ta, block b and
    // K range kk (rest = wave + W i, wave-uniform), loaded straight into LDS:
    // lane L's 16 bytes land at the tile's base + 16 L, which is the fragment
    // order (row m = L & 15, slice L >> 4). Out-of-range lanes write zeros.
    const uint64_t waddr = (uint64_t)(uintptr_t)p.P.base;
    const u32x4_t rsv = {(uint32_t)waddr, (uint32_t)(waddr >> 32) & 0xFFFFu, p.P.bytes, 0x00020000u};
    const uint32_t xlane = (uint32_t)(((int64_t)(lane & 15) * p.ldx + 8 * (lane >> 4)) * 2);
    // the activations' buffer descriptor as four dwords (base, stride 0, size,
    // the same flags as the builtin's), and the LDS address of `lds`
    const uint64_t xaddr = (uint64_t)(uintptr_t)p.x;
    const u32x4_t xrsv = {(uint32_t)xaddr, (uint32_t)(xaddr >> 32) & 0xFFFFu, x_bytes, 0x00020000u};
    const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)lds;
    auto load_x = [&](int i_local) {
        uint8_t* xb = xbase + (i_local % C::NXB) * C::XBUF;  // (step i - 1's buffer when issued at step i - 1 + NXB)
#pragma unroll
        for (int i = 0; i < C::XI; ++i) {
            const int rest = wave + C::W * i;
            const int ta = rest % NT, b = (rest / NT) % NB, kk = rest / (NT * NB);
            const int kb = (int)(((int64_t)total_steps * kk) / WK);
            const int se = (int)(((int64_t)total_steps * (kk + 1)) / WK);
            const int s = kb + i_local;
            const int kblk = s * (NB * 32) + 32 * b;  // the block's first k (K is a multiple of 32)
            const bool ok = s < se && kblk < p.K && 16 * ta + (lane & 15) < M;
            const uint32_t off = xlane + (uint32_t)(((int64_t)16 * ta * p.ldx + kblk) * 2);
            const uint32_t dst = (uint32_t)(uintptr_t)(xb + kk * C::XWIN + (b * NT + ta) * 1024 - lds) + lds_base;
            lds_load16(xrsv, oob_unless(off, ok ? 0xFFFFFFFFu : 0u), __builtin_amdgcn_readfirstlane(dst));
        }
    };
    // s_waitcnt vmcnt(n) (gfx9 encoding: vmcnt in bits 3:0 and 15:14; expcnt and
    // lgkmcnt left at their maxima, i.e. not waited on)
    constexpr int NW_LOADS = NI * QP, NX_LOADS = C::XI;
    constexpr int XWAIT = NW_LOADS + (D - 1) * (NX_LOADS + NW_LOADS);  // loads issued after a step's tiles
    static_assert(XWAIT < 64, "vmcnt holds six bits");
    constexpr int META_WAIT = D * (NX_LOADS + NW_LOADS);  // loads issued after the scale table
    static_assert(META_WAIT < 64, "vmcnt holds six bits");
    constexpr int META_WAIT_ENC = (META_WAIT & 15) | (7 << 4) | (15 << 8) | ((META_WAIT >> 4) << 14);
    constexpr int XWAIT_ENC = (XWAIT & 15) | (7 << 4) | (15 << 8) | ((XWAIT >> 4) << 14);

    // Issue order: a step's activation tiles, then its weights. The compiler
    // does not count the LDS loads when it places its waits for the weights,
    // so a wait for step i's weights (all but step i + 1's weights complete)
    // also covers step i's and step i + 1's tiles -- never later weights.
    // D + 1 weight register sets rotate with the loop unrolled by D + 1: step
    // i reads set i % (D + 1) and loads step i + D into the set step i - 1
    // read, so every set keeps its registers around the loop.
    constexpr int NS = D + 1;  // weight register sets and activation buffers in rotation
    static_assert(C::NXB == NS, "one activation buffer per weight set");
    WSet w[NS];
    {
        // the scale table, straight into LDS: piece (row r, quad q) of the
        // wave's range; surplus instructions load nothing into the dummy area
        const uint32_t lbase = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)lds;
        const uint32_t meta_l = (uint32_t)(meta - lds) + lbase, meta_dl = (uint32_t)(meta_d - lds) + lbase;
        const uint32_t dummy_l = (uint32_t)(dummy - lds) + lbase;
        const int s_used = C::s_bytes(nq_row) / C::SPI;
#pragma unroll
        for (int l = 0; l < C::MS; ++l) {
            constexpr int PPI = C::SPI / C::QB;  // pieces per instruction... (or dwords for 8-byte quads)
            int r, q, half = 0;
            if constexpr (C::QB == 16) {
                const int pi = l * 64 + lane;
                r = pi / nq_row;
                q = pi % nq_row;
            } else {  // two dwords per 8-byte quad
                const int di = l * 64 + lane;
                r = (di >> 1) / nq_row;
                q = (di >> 1) % nq_row;
                half = di & 1;
            }
            (void)PPI;
            const int gq = q_begin + q;
            int nb;
            const uint32_t off = region_of(r, gq, nb) + (uint32_t)(gq & 15) * (uint32_t)C::QB + 4u * (uint32_t)half;
            const bool ok = l < s_used && r < 16 && row0 + r < p.rows && q < nq && gq < total_quads;
            const uint32_t dst = __builtin_amdgcn_readfirstlane(l < s_used ? meta_l + (uint32_t)(l * C::SPI) : dummy_l);
            if constexpr (C::QB == 16) lds_load16(rsv, oob_unless(off, ok ? 0xFFFFFFFFu : 0u), dst);
            else lds_load4(rsv, oob_unless(off, ok ? 0xFFFFFFFFu : 0u), dst);
        }
        if constexpr (FMT == Q6_K) {
            const int d_used = C::d_bytes(nq_row) / 256;
#pragma unroll
            for (int l = 0; l < C::MD; ++l) {
                const int pi = l * 64 + lane;
                const int r = pi / nq_row, q = pi % nq_row, gq = q_begin + q;
                int nb;
                const uint32_t region = region_of(r, gq, nb);
                // the aligned dword holding quad gq's fp16 d (low half for even gq)
                const uint32_t off = region + (uint32_t)(nb >> 2) * 16u + (uint32_t)(gq & 14) * 2u;
                const bool ok = l < d_used && r < 16 && row0 + r < p.rows && q < nq && gq < total_quads;
                const uint32_t dst = __builtin_amdgcn_readfirstlane(l < d_used ? meta_dl + (uint32_t)(l * 256) : dummy_l);
                lds_load4(rsv, oob_unless(off, ok ? 0xFFFFFFFFu : 0u), dst);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < D; ++i) {
        load_x(i);
        load_w(s_begin + i, w[i]);
    }
    // Chunks past the row's end inside its last quad (Q8_0 and Q4_0 rows of a
    // chunk count not a multiple of four) hold whatever bytes follow the scale
    // region: zero their scales once the table is in, so that they add
    // nothing (their weights and activations are zeros).
    if constexpr (FMT == Q8_0 || FMT == Q4_0) {
        __builtin_amdgcn_s_waitcnt(META_WAIT_ENC);
        const int last = total_quads - 1 - q_begin;
        if ((nch & 3) && last >= 0 && last < nq && lane < 16) {
            uint8_t* piece = meta + (lane * nq_row + last) * C::QB;
            for (int c = nch & 3; c < 4; ++c) {
                if constexpr (FMT == Q8_0) *reinterpret_cast<uint16_t*>(piece + 2 * c) = 0;
                else *reinterpret_cast<uint32_t*>(piece + 4 * c) = 0;
            }
        }
    }

    f4_t acc[NT];
#pragma unroll
    for (int ta = 0; ta < NT; ++ta) acc[ta] = f4_t{0.f, 0.f, 0.f, 0.f};

    const uint8_t* my_meta = meta + mn * nq_row * C::QB;                       // the scales of this lane's row n
    const uint32_t* my_d = reinterpret_cast<const uint32_t*>(meta_d) + mn * nq_row;  // (Q6_K)
    const int xoff = wk * C::XWIN + lane * 16;

    // B-operand words of every block of a step (after the transposes):
    // Q4_0 / Q4_K: X0, X1 = code parts 0 and 1; Q8_0: X0, X1 = the even and odd
    // words of each slice; Q6_K: X0, X1 = the low-nibble parts, X2, X3 = the
    // high fields of the slice's scale group in blocks 0 and 1 of each chunk.
    struct BWords {
        uint32_t X0[NI][4], X1[NI][4], X2[NI][4], X3[NI][4];
    };
    auto prepare = [&](const WSet& wv, BWords& bw) {
        if constexpr (FMT == Q8_0) {
            // slice kq = words 2kq, 2kq+1 of the 32-weight chunk: part j >> 1,
            // word 2 (j & 1) (+1), transposed apart
#pragma unroll
            for (int h = 0; h < NI; ++h)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    bw.X0[h][j] = wv[j >> 1][h][2 * (j & 1)];
                    bw.X1[h][j] = wv[j >> 1][h][2 * (j & 1) + 1];
                }
        } else {
#pragma unroll
            for (int h = 0; h < NI; ++h)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    bw.X0[h][j] = wv[0][h][j];
                    bw.X1[h][j] = wv[1][h][j];
                    if constexpr (FMT == Q6_K) {
                        // lane kq wants the high fields of scale group 2 sub + kq / 2
                        bw.X2[h][j] = wv[2][h][j >> 1];
                        bw.X3[h][j] = wv[2][h][2 + (j >> 1)];
                    }
                }
        }
        transpose_words<RB>(bw.X0, lane);
        transpose_words<RB>(bw.X1, lane);
        if constexpr (FMT == Q6_K) {
            transpose_words<RB>(bw.X2, lane);
            transpose_words<RB>(bw.X3, lane);
        }
    };

    uint32_t vmask = 0x00F0000Fu, vmagic = 0x54006400u;
    asm volatile("" : "+v"(vmask), "+v"(vmagic));
    auto multiply = [&](const BWords& bw, const uint8_t* xb, int i_local) {
        constexpr int NQ = CPS / 4;               // quads (of scales) per step
        const int qrel = i_local * NQ;            // first quad of the step within the wave's range
        // -- every LDS read of the step first, so their latencies overlap --
        h8_t A[NB][NT];
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int ta = 0; ta < NT; ++ta) A[b][ta] = *reinterpret_cast<const h8_t*>(xb + xoff + (b * NT + ta) * 1024);
        uint4 mq[NQ];
        float dq[NQ];
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            const int quad = min(qrel + q, nq_row - 1);
            if constexpr (F::QB == 16) {
                mq[q] = *reinterpret_cast<const uint4*>(my_meta + quad * 16);
            } else {
                const uint2 v = *reinterpret_cast<const uint2*>(my_meta + quad * 8);
                mq[q] = make_uint4(v.x, v.y, 0u, 0u);
            }
            if constexpr (FMT == Q6_K) {
                const uint32_t dw = my_d[quad];
                dq[q] = ((q_begin + quad) & 1) ? half_hi(dw) : half_lo(dw);
            } else {
                dq[q] = 0.f;
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        // -- the B operands of every block --
        h8_t Bf[NB], B0f[FMT == Q6_K ? NB : 1];
#pragma unroll
        for (int c = 0; c < CPS; ++c)
#pragma unroll
            for (int sub = 0; sub < F::BPC; ++sub) {
                const int b = c * F::BPC + sub;
                uint32_t o[4];
                if constexpr (FMT == Q4_0 || FMT == Q4_K) {
                    const uint32_t neg = FMT == Q4_0 ? 0xD480E408u : 0xD400E400u;
                    nibbles_to_h_v(tword<RB>(sub ? bw.X1 : bw.X0, c) ^ 0x88888888u, neg, vmask, vmagic, o);
                } else if constexpr (FMT == Q8_0) {
                    bytes_to_h(tword<RB>(bw.X0, c), o[0], o[1]);
                    bytes_to_h(tword<RB>(bw.X1, c), o[2], o[3]);
                } else {
                    const uint32_t L = tword<RB>(sub ? bw.X1 : bw.X0, c) ^ 0x88888888u;
                    const uint32_t H = tword<RB>(sub ? bw.X3 : bw.X2, c);
                    q6_to_h(L, (H >> (2 * (kq & 1))) & 0x33333333u, o);
                }
                Bf[b] = __builtin_bit_cast(h8_t, make_uint4(o[0], o[1], o[2], o[3]));
                if constexpr (FMT == Q6_K) {
                    // a block's slices 0, 1 are scale group 2 sub, slices 2, 3
                    // group 2 sub + 1: the block's product and its first
                    // group's (the second group's weights zeroed) give both sums
                    const bool g0 = kq < 2;
                    B0f[b] = __builtin_bit_cast(h8_t, make_uint4(g0 ? o[0] : 0u, g0 ? o[1] : 0u, g0 ? o[2] : 0u, g0 ? o[3] : 0u));
                }
            }
        // -- every product of the step, then the scaled sums (so that no sum
        //    waits on the product issued just before it) --
        constexpr int NP = FMT == Q6_K || FMT == Q4_K ? 2 : 1;  // products per block and tile
        f4_t Dv[NB][NT][NP];
        const f4_t z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int ta = 0; ta < NT; ++ta) {
                Dv[b][ta][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[b][ta], Bf[b], z, 0, 0, 0);
                if constexpr (FMT == Q6_K) {
                    Dv[b][ta][NP - 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[b][ta], B0f[b], z, 0, 0, 0);
                } else if constexpr (FMT == Q4_K) {
                    const h8_t one = {1, 1, 1, 1, 1, 1, 1, 1};
                    Dv[b][ta][NP - 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[b][ta], one, z, 0, 0, 0);
                }
            }
#pragma unroll
        for (int c = 0; c < CPS; ++c) {
            // (chunks past the row or the wave's range add nothing: their
            // activations are zeros and their scales zero or finite)
            const uint4& m4 = mq[c / 4];
            float s[2] = {0.f, 0.f}, mnv[2] = {0.f, 0.f}, s6[4] = {0.f, 0.f, 0.f, 0.f};
            if constexpr (FMT == Q4_K) {
                uint32_t sc0, m0, sc1, m1;
                q4k_scales(m4, c & 3, sc0, m0, sc1, m1);
                const float dd = half_lo(m4.x), dmin = half_hi(m4.x);
                s[0] = dd * (float)sc0;
                s[1] = dd * (float)sc1;
                mnv[0] = dmin * (float)m0;
                mnv[1] = dmin * (float)m1;
            } else if constexpr (FMT == Q4_0) {
                const uint32_t dw = word(m4, c & 3);
                s[0] = half_lo(dw);
                s[1] = half_hi(dw);
            } else if constexpr (FMT == Q8_0) {
                const uint32_t dw = word(m4, (c & 3) >> 1);
                s[0] = (c & 1) ? half_hi(dw) : half_lo(dw);
            } else {
                const uint32_t scw = word(m4, c & 3);
#pragma unroll
                for (int g = 0; g < 4; ++g) s6[g] = dq[c / 4] * (float)(int8_t)((scw >> (8 * g)) & 0xffu);
            }
#pragma unroll
            for (int sub = 0; sub < F::BPC; ++sub) {
                const int b = c * F::BPC + sub;
#pragma unroll
                for (int ta = 0; ta < NT; ++ta) {
                    if constexpr (FMT == Q6_K) {
                        // s0 D0 + s1 (Da - D0) = (s0 - s1) D0 + s1 Da
                        const float s01 = s6[2 * sub] - s6[2 * sub + 1];
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            acc[ta][j] = fmaf(s6[2 * sub + 1], Dv[b][ta][0][j], fmaf(s01, Dv[b][ta][NP - 1][j], acc[ta][j]));
                    } else if constexpr (FMT == Q4_K) {
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            acc[ta][j] = fmaf(-mnv[sub], Dv[b][ta][NP - 1][j], fmaf(s[sub], Dv[b][ta][0][j], acc[ta][j]));
                    } else {
#pragma unroll
                        for (int j = 0; j < 4; ++j) acc[ta][j] = fmaf(s[sub], Dv[b][ta][0][j], acc[ta][j]);
                    }
                }
            }
        }
    };

    // Main loop: at step i (local), wait for its loads, issue step i + D's into
    // the same register slot after its words are copied out, stage its
    // activations, and multiply after the barrier. Whole rounds of D steps; the
    // steps past the range load nothing and add zero.
    const int rounds = (steps_per_wave + NS - 1) / NS;
    for (int r = 0; r < rounds; ++r) {
#pragma unroll
        for (int u = 0; u < NS; ++u) {
            const int i = r * NS + u;
            // (steps past the range, up to D in the last round, load nothing and add zero)
            BWords bw;
            prepare(w[u], bw);
            // the transposes stay before the next step's loads: their wait for
            // step i's weights then counts no later load
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_waitcnt(XWAIT_ENC);  // this wave's tiles of step i are in LDS
            __syncthreads();                         // ... and every wave's; step i - 1's reads are done
            load_x(i + D);                           // into the buffer step i - 1 used
            load_w(s_begin + i + D, w[(u + D) % NS]);
            multiply(bw, xbase + u * C::XBUF, i);
        }
    }

    // no load may still be writing LDS past this point (the tail steps' tiles)
    __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));  // vmcnt(0)

    // ---- partial sums of the K ranges, in order ----
    if constexpr (WK > 1) {
        __syncthreads();
        f4_t* red = reinterpret_cast<f4_t*>(lds);
#pragma unroll
        for (int ta = 0; ta < NT; ++ta) red[((wk * WR + wr) * NT + ta) * 64 + lane] = acc[ta];
        __syncthreads();
        if (wk != 0) return;
#pragma unroll
        for (int ta = 0; ta < NT; ++ta) {
            f4_t t = red[((0 * WR + wr) * NT + ta) * 64 + lane];
#pragma unroll
            for (int v = 1; v < WK; ++v) {
                const f4_t o = red[((v * WR + wr) * NT + ta) * 64 + lane];
#pragma unroll
                for (int j = 0; j < 4; ++j) t[j] += o[j];
            }
            acc[ta] = t;
        }
    }
    const int64_t row = row0 + mn;
    if (row < p.rows) {
#pragma unroll
        for (int ta = 0; ta < NT; ++ta)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int m = 16 * ta + 4 * kq + j;
                if (m < M) p.y[(int64_t)m * p.ldy + row] = acc[ta][j];
            }
    }
}

}  // namespace rq
