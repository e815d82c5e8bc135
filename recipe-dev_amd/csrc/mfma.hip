// Small-M quantized products on the matrix cores: launch planning and the
// fp16-activation kernels (the kernels themselves are in mfma_impl.h).
#include "mfma_impl.h"
#include "mfma_rt.h"

namespace rq {

// ---- streaming form (mfma_rt.h) ----
template <int FMT, int RB, int NT, int WR, int WK>
static hipError_t launch_rt_one(const MvParams& p, int M, uint32_t x_bytes, hipStream_t stream, hipEvent_t ev0,
                                hipEvent_t ev1) {
    const int ys = (M + 16 * NT - 1) / (16 * NT);  // activation row groups (grid y)
    using C = RtCfg<FMT, RB, NT, WR, WK>;
    const int total_steps = (p.P.nch + C::CPS - 1) / C::CPS;
    const int spw = (total_steps + WK - 1) / WK;
    const int quads = spw * C::CPS / 4;
    const size_t lds = (size_t)C::lds_bytes(quads);
    if (quads > kRtMaxQuads || lds > 160 * 1024) return hipErrorNotSupported;
    auto kernel = matvec_mfma_rt<FMT, RB, NT, WR, WK>;
    if (lds > 65536) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    const int64_t tiles = (p.rows + 15) / 16;
    const int grid = (int)((tiles + WR - 1) / WR);
    if (ev0 || ev1)
        hipExtLaunchKernelGGL(kernel, dim3(grid, ys), dim3(64 * WR * WK), (uint32_t)lds, stream, ev0, ev1, 0u, p, M,
                              x_bytes, spw);
    else
        hipLaunchKernelGGL(kernel, dim3(grid, ys), dim3(64 * WR * WK), lds, stream, p, M, x_bytes, spw);
    return hipGetLastError();
}

// LDS of a launch shape, for choosing the step (0 if the K range does not fit).
template <int FMT, int RB, int NT, int WR, int WK>
static size_t rt_lds(const MvParams& p) {
    using C = RtCfg<FMT, RB, NT, WR, WK>;
    const int total_steps = (p.P.nch + C::CPS - 1) / C::CPS;
    const int quads = (total_steps + WK - 1) / WK * C::CPS / 4;
    return quads > kRtMaxQuads ? 0 : (size_t)C::lds_bytes(quads);
}

template <int FMT, int NT, int WR, int WK>
static hipError_t launch_rt_w(const MvParams& p, int M, uint32_t x_bytes, hipStream_t stream, hipEvent_t ev0,
                              hipEvent_t ev1) {
    // whole 128-byte runs per row (RB = 8) while two workgroups still fit a CU
    const char* env = getenv("RQMV_RT_RB");
    const int want = env && *env ? atoi(env) : 0;
    if constexpr (NT == 1 && WR >= 2 && FMT != Q6_K) {  // (the others need too many registers)
        const size_t l8 = rt_lds<FMT, 8, NT, WR, WK>(p);
        if (want != 16 && l8 && (want == 8 || l8 <= 80 * 1024))
            return launch_rt_one<FMT, 8, NT, WR, WK>(p, M, x_bytes, stream, ev0, ev1);
    }
    (void)want;
    return launch_rt_one<FMT, 16, NT, WR, WK>(p, M, x_bytes, stream, ev0, ev1);
}

// Workgroup shape (WR row tiles x WK K ranges), from the units of work (row
// tiles x activation row groups) against the CUs. Measured on MI355X (kernel
// us, fp16 x):
//   four row tiles per workgroup once there are units for three waves per CU:
//     Q4_K 4096->14336 at 32 rows (896 tiles) 34.8 (2 x 2) -> 25.3,
//   with two K ranges each below six (8 waves per workgroup): the same at
//     16 rows 19.7 -> 18.6;
//   split K four ways for long rows on few units: Q4_K 14336->4096 at 16 rows
//     26.2 (2 x 2: 33.4); with the rows split in two, 2 x 2 (33.3; 4 K ranges
//     50.9);
//   Q8_0 with its rows split in two: four row tiles (Q8_0 5120x5120 at 32 rows
//     24.4 -> 20.5);
//   else two tiles x two K ranges.
// RQMV_RT_SHAPE ("41", "42", "22" or "14") overrides it for tuning.
template <int FMT, int NT>
static hipError_t launch_rt(const MvParams& p, int M, uint32_t x_bytes, int cus, int ys, hipStream_t stream,
                            hipEvent_t ev0, hipEvent_t ev1) {
    const int64_t units = (p.rows + 15) / 16 * ys;
    const char* env = getenv("RQMV_RT_SHAPE");
    int shape;
    if (env && *env) shape = atoi(env);
    else if (units >= (int64_t)6 * cus) shape = 41;
    else if (units >= (int64_t)3 * cus) shape = NT == 1 ? 42 : 41;
    else if (FMT == Q8_0 && ys > 1) shape = 41;
    else if (p.K > 8192 && units < (int64_t)2 * cus) shape = 14;
    else shape = 22;
    // split K four ways stages four activation windows per workgroup: for two
    // tiles of 32-weight blocks of 64-weight chunks that is too many registers
    if (NT == 2 && FMT != Q8_0 && shape == 14) shape = 22;
    if (NT == 2 && shape == 42) shape = 41;
    hipError_t e = hipErrorNotSupported;
    if constexpr (NT == 1)
        if (shape == 42) e = launch_rt_w<FMT, NT, 4, 2>(p, M, x_bytes, stream, ev0, ev1);
    if (shape == 41 || (shape == 42 && e == hipErrorNotSupported)) e = launch_rt_w<FMT, NT, 4, 1>(p, M, x_bytes, stream, ev0, ev1);
    if (e == hipErrorNotSupported && shape >= 22) e = launch_rt_w<FMT, NT, 2, 2>(p, M, x_bytes, stream, ev0, ev1);
    if constexpr (NT == 1 || FMT == Q8_0)
        if (e == hipErrorNotSupported) e = launch_rt_w<FMT, NT, 1, 4>(p, M, x_bytes, stream, ev0, ev1);
    return e;
}

// More than 16 activation rows: two 16-row tiles per wave (NT = 2), or, when
// the row tiles are too few to give every CU two, the 16-row form on two
// workgroup rows, one per half: twice the waves, each decoding the weights
// for its half, which the second reads from the caches. Measured: Q8_0
// 5120x5120 at 32 rows 24.4 -> 20.5 us, Q4_K 14336->4096 47.6 -> 33.3, Q4_K
// 4096x4096 18.1 -> 13.8; with plenty of tiles it loses (Q4_K 4096->14336
// 25.3 -> 28.6, Q6_K 5120->25600 56.3 -> 80.5). RQMV_RT_MSPLIT=0/1 forces
// either.
template <int FMT>
static hipError_t launch_rt_fmt(const MvParams& p, int M, uint32_t x_bytes, int cus, hipStream_t stream, hipEvent_t ev0,
                                hipEvent_t ev1) {
    if (M <= 16) return launch_rt<FMT, 1>(p, M, x_bytes, cus, 1, stream, ev0, ev1);
    const char* env = getenv("RQMV_RT_MSPLIT");
    const bool split = env && *env ? *env != '0' : (p.rows + 15) / 16 < (int64_t)2 * cus;
    if (split) return launch_rt<FMT, 1>(p, M, x_bytes, cus, 2, stream, ev0, ev1);
    return launch_rt<FMT, 2>(p, M, x_bytes, cus, 1, stream, ev0, ev1);
}

template <int FMT>
static hipError_t launch_mfma_sk(const MvParams& p, int M, uint32_t x_bytes, hipStream_t stream, hipEvent_t ev0,
                                 hipEvent_t ev1) {
    const size_t lds = SkLds<FMT>::TOTAL;
    auto kernel = matvec_mfma_sk<FMT>;
    const int grid = (int)((p.rows + 15) / 16);
    if (ev0 || ev1)
        hipExtLaunchKernelGGL(kernel, dim3(grid), dim3(64 * kSplitK), (uint32_t)lds, stream, ev0, ev1, 0u, p, M, x_bytes);
    else
        hipLaunchKernelGGL(kernel, dim3(grid), dim3(64 * kSplitK), lds, stream, p, M, x_bytes);
    return hipGetLastError();
}

template <int FMT>
static size_t lds_of(bool f32, bool two, int W) {
    if (W == 1 && (f32 || two)) W = 2;  // as launch_mfma_w
#define RQ_LDS(NT, XF) (W == 1 ? MfmaLds<FMT, NT, XF, 1>::TOTAL : W == 2 ? MfmaLds<FMT, NT, XF, 2>::TOTAL : MfmaLds<FMT, NT, XF, 4>::TOTAL)
    return two ? (f32 ? RQ_LDS(2, true) : RQ_LDS(2, false)) : (f32 ? RQ_LDS(1, true) : RQ_LDS(1, false));
#undef RQ_LDS
}

// Waves (16-row stripes) per workgroup: four when there are rows enough to
// give every CU a few workgroups, fewer for short matrices. RQMV_MFMA_WAVES
// overrides it for tuning.
static int mfma_waves(int64_t rows, int cus) {
    const int64_t stripes = (rows + 15) / 16;
    const char* env = getenv("RQMV_MFMA_WAVES");
    if (env && *env) {
        const int w = atoi(env);
        if (w == 1 || w == 2 || w == 4) return w;
    }
    if (stripes >= (int64_t)6 * cus) return 4;
    if (stripes >= (int64_t)3 * cus) return 2;
    return 1;
}

size_t mfma_lds_bytes(int fmt, int xtype, int M, int64_t rows, int cus) {
    const bool f32 = xtype == X_F32, two = M > 16;
    if (!two && !f32) {
        const size_t sk = fmt == Q4_0 ? SkLds<Q4_0>::TOTAL : fmt == Q4_K ? SkLds<Q4_K>::TOTAL
                        : fmt == Q8_0 ? SkLds<Q8_0>::TOTAL : fmt == Q6_K ? SkLds<Q6_K>::TOTAL : 0;
        if (sk) return sk;  // (the larger of the two forms is below the LDS limit either way)
    }
    const int W = mfma_waves(rows, cus);
    switch (fmt) {
        case Q4_0: return lds_of<Q4_0>(f32, two, W);
        case Q4_K: return lds_of<Q4_K>(f32, two, W);
        case Q8_0: return lds_of<Q8_0>(f32, two, W);
        case Q6_K: return lds_of<Q6_K>(f32, two, W);
        default: return 0;
    }
}

// fp32 activations (mfma_f32.hip: built without the matrix-core VGPR form,
// which the per-block power-of-two epilogue of that path does not compile under).
hipError_t launch_mfma_f32(int fmt, bool two, int W, const MvParams& p, int M, uint32_t x_bytes, hipStream_t stream,
                           hipEvent_t ev0, hipEvent_t ev1);

template <int FMT>
static hipError_t launch_mfma_fmt(int xtype, int W, const MvParams& p, int M, uint32_t x_bytes, hipStream_t stream,
                                  hipEvent_t ev0, hipEvent_t ev1) {
    if (xtype == X_F32) return launch_mfma_f32(FMT, M > 16, W, p, M, x_bytes, stream, ev0, ev1);
    if (M > 16) return launch_mfma_w<FMT, 2, false>(W, p, M, x_bytes, stream, ev0, ev1);
    return launch_mfma_w<FMT, 1, false>(W, p, M, x_bytes, stream, ev0, ev1);
}

hipError_t launch_matvec_mfma(int fmt, int xtype, int M, const MvParams& p, int cus, hipStream_t stream,
                              hipEvent_t ev0, hipEvent_t ev1) {
    if (M < 1 || M > 32) return hipErrorInvalidValue;
    const size_t esize = xtype == X_F32 ? 4 : 2;
    const int64_t x_bytes = ((int64_t)(M - 1) * p.ldx + p.K) * (int64_t)esize;
    if (x_bytes >= (int64_t)kOobOffset) return hipErrorInvalidValue;
    // fp16 activations: the streaming form, unless its scale table does not
    // fit (K ranges longer than it holds) or RQMV_MFMA_RT=0 asks for the
    // staged forms below.
    const char* rt_env = getenv("RQMV_MFMA_RT");
    // (long rows on few row tiles, at most 16 activation rows: the split-K form,
    // whose waves read their activation fragments from the caches, measured
    // faster: Q4_K 14336->4096 at 16 rows 26.4 -> 24.1 us)
    const bool long_few = M <= 16 && p.K > 8192 && (p.rows + 15) / 16 < (int64_t)2 * cus;
    if (xtype == X_F16 && !(rt_env && *rt_env == '0') && !(long_few && !(rt_env && *rt_env == '1'))) {
        hipError_t e = hipErrorInvalidValue;
        switch (fmt) {
            case Q4_0: e = launch_rt_fmt<Q4_0>(p, M, (uint32_t)x_bytes, cus, stream, ev0, ev1); break;
            case Q4_K: e = launch_rt_fmt<Q4_K>(p, M, (uint32_t)x_bytes, cus, stream, ev0, ev1); break;
            case Q8_0: e = launch_rt_fmt<Q8_0>(p, M, (uint32_t)x_bytes, cus, stream, ev0, ev1); break;
            case Q6_K: e = launch_rt_fmt<Q6_K>(p, M, (uint32_t)x_bytes, cus, stream, ev0, ev1); break;
            default: break;
        }
        if (e != hipErrorNotSupported) return e;
    }
    // Split-K for short and medium matrices (each wave re-reads its
    // activations from the caches, which pays off while the stripes are too
    // few to fill the GPU); the shared-staging form for tall ones.
    // RQMV_MFMA_SK=0/1 forces either.
    const char* sk_env = getenv("RQMV_MFMA_SK");
    const bool sk = sk_env && *sk_env ? *sk_env != '0' : (p.rows + 15) / 16 <= (int64_t)4 * cus;
    if (M <= 16 && xtype == X_F16 && sk) {
        switch (fmt) {
            case Q4_0: return launch_mfma_sk<Q4_0>(p, M, (uint32_t)x_bytes, stream, ev0, ev1);
            case Q4_K: return launch_mfma_sk<Q4_K>(p, M, (uint32_t)x_bytes, stream, ev0, ev1);
            case Q8_0: return launch_mfma_sk<Q8_0>(p, M, (uint32_t)x_bytes, stream, ev0, ev1);
            case Q6_K: return launch_mfma_sk<Q6_K>(p, M, (uint32_t)x_bytes, stream, ev0, ev1);
            default: return hipErrorInvalidValue;
        }
    }
    const int W = mfma_waves(p.rows, cus);
    switch (fmt) {
        case Q4_0: return launch_mfma_fmt<Q4_0>(xtype, W, p, M, (uint32_t)x_bytes, stream, ev0, ev1);
        case Q4_K: return launch_mfma_fmt<Q4_K>(xtype, W, p, M, (uint32_t)x_bytes, stream, ev0, ev1);
        case Q8_0: return launch_mfma_fmt<Q8_0>(xtype, W, p, M, (uint32_t)x_bytes, stream, ev0, ev1);
        case Q6_K: return launch_mfma_fmt<Q6_K>(xtype, W, p, M, (uint32_t)x_bytes, stream, ev0, ev1);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace rq

