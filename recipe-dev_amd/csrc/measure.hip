// Measurement kernels for bench.py, built as libmeasure.so beside librqmv.so
// (not part of the product library): a plain streaming read of a device
// buffer at a chosen grid, the bandwidth reference that a matrix-vector
// launch is read against (the same bytes, the same grid, one launch); and an
// issue-rate probe of single VALU opcodes, which the kernels' choice of
// instructions rests on.
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

// Issue-rate probe: eight independent chains of one VALU opcode per lane
// (inline assembly, so the opcode is exactly the one named), `iters` rounds;
// the chains' xor goes to out[gid]. With 2,048 workgroups of 256 threads
// (eight waves per SIMD) the SIMDs issue back to back, and a launch's time
// over its wave-instructions per SIMD is the opcode's issue cost.
#define RQ_CHAIN8(ASM)                                       \
    for (int i = 0; i < iters; ++i) {                        \
        asm volatile(ASM : "+v"(a0) : "v"(b), "v"(c));       \
        asm volatile(ASM : "+v"(a1) : "v"(b), "v"(c));       \
        asm volatile(ASM : "+v"(a2) : "v"(b), "v"(c));       \
        asm volatile(ASM : "+v"(a3) : "v"(b), "v"(c));       \
        asm volatile(ASM : "+v"(a4) : "v"(b), "v"(c));       \
        asm volatile(ASM : "+v"(a5) : "v"(b), "v"(c));       \
        asm volatile(ASM : "+v"(a6) : "v"(b), "v"(c));       \
        asm volatile(ASM : "+v"(a7) : "v"(b), "v"(c));       \
    }
#define RQ_ISSUE_KERNEL(NAME, ASM)                                                                        \
    __global__ void __launch_bounds__(256) NAME(uint32_t* out, uint32_t seed, int iters) {                 \
        uint32_t a0 = threadIdx.x ^ seed, a1 = a0 + 1, a2 = a0 + 2, a3 = a0 + 3, a4 = a0 + 4, a5 = a0 + 5, \
                 a6 = a0 + 6, a7 = a0 + 7;                                                                  \
        const uint32_t b = 0x3c003c00u ^ (seed & 1), c = 0x01010101u + (seed >> 8);                        \
        RQ_CHAIN8(ASM)                                                                                      \
        out[blockIdx.x * 256 + threadIdx.x] = a0 ^ a1 ^ a2 ^ a3 ^ a4 ^ a5 ^ a6 ^ a7;                      \
    }
RQ_ISSUE_KERNEL(issue_add_u32, "v_add_u32 %0, %1, %0")
RQ_ISSUE_KERNEL(issue_and_b32, "v_and_b32 %0, %1, %0")
RQ_ISSUE_KERNEL(issue_lshrrev_b32, "v_lshrrev_b32 %0, 4, %0")
RQ_ISSUE_KERNEL(issue_mov_b32, "v_mov_b32 %0, %1")
RQ_ISSUE_KERNEL(issue_mul_f32, "v_mul_f32 %0, %1, %0")
RQ_ISSUE_KERNEL(issue_fmac_f32, "v_fmac_f32 %0, %1, %2")
RQ_ISSUE_KERNEL(issue_fma_f32, "v_fma_f32 %0, %1, %2, %0")
RQ_ISSUE_KERNEL(issue_bfe_u32, "v_bfe_u32 %0, %0, 4, 6")
RQ_ISSUE_KERNEL(issue_perm_b32, "v_perm_b32 %0, %1, %0, %2")
RQ_ISSUE_KERNEL(issue_and_or_b32, "v_and_or_b32 %0, %0, %1, %2")
RQ_ISSUE_KERNEL(issue_lshl_or_b32, "v_lshl_or_b32 %0, %0, 4, %1")
RQ_ISSUE_KERNEL(issue_cvt_f32_i32, "v_cvt_f32_i32 %0, %0")
RQ_ISSUE_KERNEL(issue_dot8_i32_i4, "v_dot8_i32_i4 %0, %1, %2, %0")
RQ_ISSUE_KERNEL(issue_dot4_i32_i8, "v_dot4_i32_i8 %0, %1, %2, %0")
RQ_ISSUE_KERNEL(issue_dot2_f32_f16, "v_dot2_f32_f16 %0, %1, %2, %0")
RQ_ISSUE_KERNEL(issue_pk_fma_f16, "v_pk_fma_f16 %0, %1, %2, %0")
#undef RQ_ISSUE_KERNEL
#undef RQ_CHAIN8

typedef void (*issue_fn)(uint32_t*, uint32_t, int);
const issue_fn kIssueKernels[] = {issue_add_u32,      issue_and_b32,      issue_lshrrev_b32, issue_mov_b32,
                                  issue_mul_f32,      issue_fmac_f32,     issue_fma_f32,     issue_bfe_u32,
                                  issue_perm_b32,     issue_and_or_b32,   issue_lshl_or_b32, issue_cvt_f32_i32,
                                  issue_dot8_i32_i4,  issue_dot4_i32_i8,  issue_dot2_f32_f16, issue_pk_fma_f16};
const char* const kIssueNames[] = {"v_add_u32",     "v_and_b32",      "v_lshrrev_b32",  "v_mov_b32",
                                   "v_mul_f32",     "v_fmac_f32",     "v_fma_f32",      "v_bfe_u32",
                                   "v_perm_b32",    "v_and_or_b32",   "v_lshl_or_b32",  "v_cvt_f32_i32",
                                   "v_dot8_i32_i4", "v_dot4_i32_i8",  "v_dot2_f32_f16", "v_pk_fma_f16"};
constexpr int kIssueOps = sizeof(kIssueKernels) / sizeof(kIssueKernels[0]);

}  // namespace

extern "C" {

// The issue-rate probe's opcodes: their count, and the name of opcode `op`.
int measure_issue_ops() { return kIssueOps; }
const char* measure_issue_name(int op) { return op >= 0 && op < kIssueOps ? kIssueNames[op] : nullptr; }

// One launch of opcode `op`'s probe: `blocks` workgroups of 256 threads,
// `iters` rounds of eight instructions per lane; `out` holds blocks * 256
// words. start/stop (hipEvent_t, may be NULL) are recorded by the dispatch.
int measure_issue_rate(int op, int blocks, int iters, uint32_t* out, void* stream, void* start, void* stop) {
    if (op < 0 || op >= kIssueOps || blocks < 1 || iters < 1 || !out) return (int)hipErrorInvalidValue;
    hipExtLaunchKernelGGL(kIssueKernels[op], dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                          static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop), 0u, out, 7u, iters);
    return (int)hipGetLastError();
}

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
