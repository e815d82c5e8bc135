// Measurement kernel for bench.py, built as libmeasure.so beside librqmv.so
// (not part of the product library): a plain streaming read of a device
// buffer at a chosen grid, the bandwidth reference that a matrix-vector
// launch is read against (the same bytes, the same grid, one launch).
#include <hip/hip_ext.h>
#include <stdint.h>

namespace {

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// Thread t of the grid reads the 16-byte units t, t + T, t + 2T, ... (T
// threads), INF of them requested before any is folded into the thread's
// xor, so that INF loads per thread are in flight. The xor goes to
// sink[gid] only when it equals `never` (a value the host picks so that no
// thread matches it), which keeps every load live and writes nothing.
template <int INF>
__global__ void __launch_bounds__(256) stream_read(const u32x4_t* __restrict__ src, uint64_t n16, uint32_t never,
                                                   uint32_t* sink) {
    const uint64_t T = (uint64_t)gridDim.x * blockDim.x;
    const uint64_t gid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint64_t u = gid;
    uint32_t acc = 0;
    for (; u + (INF - 1) * T < n16; u += INF * T) {
        u32x4_t v[INF];
#pragma unroll
        for (int i = 0; i < INF; ++i) v[i] = __builtin_nontemporal_load(src + u + i * T);
#pragma unroll
        for (int i = 0; i < INF; ++i) acc ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    }
    for (; u < n16; u += T) {
        const u32x4_t v = __builtin_nontemporal_load(src + u);
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == never) sink[gid] = acc;
}

}  // namespace

extern "C" {

// Reads `bytes` (a multiple of 16) at `src` with `grid` workgroups of 256
// threads and `inflight` (1, 2, 4 or 8) loads in flight per thread; `sink`
// holds grid * 256 words. start/stop (hipEvent_t, may be NULL) are recorded
// by the dispatch itself. Returns 0, or a HIP error code.
int measure_stream_read(const void* src, uint64_t bytes, int grid, int inflight, uint32_t never, uint32_t* sink,
                        void* stream, void* start, void* stop) {
    if (!src || !sink || grid < 1 || bytes % 16) return (int)hipErrorInvalidValue;
    const uint64_t n16 = bytes / 16;
    auto s = static_cast<hipStream_t>(stream);
    auto e0 = static_cast<hipEvent_t>(start), e1 = static_cast<hipEvent_t>(stop);
    const u32x4_t* p = static_cast<const u32x4_t*>(src);
    switch (inflight) {
        case 1: hipExtLaunchKernelGGL(stream_read<1>, dim3(grid), dim3(256), 0, s, e0, e1, 0u, p, n16, never, sink); break;
        case 2: hipExtLaunchKernelGGL(stream_read<2>, dim3(grid), dim3(256), 0, s, e0, e1, 0u, p, n16, never, sink); break;
        case 4: hipExtLaunchKernelGGL(stream_read<4>, dim3(grid), dim3(256), 0, s, e0, e1, 0u, p, n16, never, sink); break;
        case 8: hipExtLaunchKernelGGL(stream_read<8>, dim3(grid), dim3(256), 0, s, e0, e1, 0u, p, n16, never, sink); break;
        default: return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}

}  // extern "C"
