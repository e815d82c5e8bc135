// Small-M quantized products on the matrix cores for fp32 activations (the
// kernels are in mfma_impl.h). Built without the matrix-core VGPR form: the
// per-block power-of-two epilogue of the fp32 path does not compile under it.
#include "mfma_impl.h"

namespace rq {

template <int FMT>
static hipError_t f32_fmt(bool two, int W, const MvParams& p, int M, uint32_t x_bytes, hipStream_t stream,
                          hipEvent_t ev0, hipEvent_t ev1) {
    if (two) return launch_mfma_w<FMT, 2, true>(W, p, M, x_bytes, stream, ev0, ev1);
    return launch_mfma_w<FMT, 1, true>(W, p, M, x_bytes, stream, ev0, ev1);
}

hipError_t launch_mfma_f32(int fmt, bool two, int W, const MvParams& p, int M, uint32_t x_bytes, hipStream_t stream,
                           hipEvent_t ev0, hipEvent_t ev1) {
    switch (fmt) {
        case Q4_0: return f32_fmt<Q4_0>(two, W, p, M, x_bytes, stream, ev0, ev1);
        case Q4_K: return f32_fmt<Q4_K>(two, W, p, M, x_bytes, stream, ev0, ev1);
        case Q8_0: return f32_fmt<Q8_0>(two, W, p, M, x_bytes, stream, ev0, ev1);
        case Q6_K: return f32_fmt<Q6_K>(two, W, p, M, x_bytes, stream, ev0, ev1);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace rq
