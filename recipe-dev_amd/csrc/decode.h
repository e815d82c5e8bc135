// Decode-step kernels around the quantized projections (decode.hip).
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

namespace rq {

hipError_t launch_add_rmsnorm(float* x, const float* delta, const float* w, int n, float eps, float* out,
                              hipStream_t stream);
hipError_t launch_rope_kv(float* qkv, const int* pos, int nq, int nkv, int hd, double base, __half* kc, __half* vc,
                          int max_ctx, hipStream_t stream);
size_t attention_workspace_bytes(int nq, int hd, int max_ctx);
hipError_t launch_attention(const float* q, const __half* kc, const __half* vc, const int* pos, int nq, int nkv,
                            int hd, int max_ctx, void* workspace, float* out, hipStream_t stream);
hipError_t launch_attention_rope(const float* qkv, const float2* rope_table, __half* kc, __half* vc, const int* pos,
                                 int nq, int nkv, int hd, int max_ctx, void* workspace, float* out,
                                 hipStream_t stream);
hipError_t launch_rope_table(float2* table, int head_dim, double base, int rows, hipStream_t stream);
hipError_t launch_silu_mul(const float* gu, int n, float* out, hipStream_t stream);
size_t argmax_workspace_bytes();
hipError_t launch_argmax(const float* v, int n, int* out, void* workspace, hipStream_t stream);
hipError_t launch_embed_row(const float* table, int rows, int n, const int* token, float* out, hipStream_t stream);
hipError_t launch_advance(int* pos, hipStream_t stream);

}  // namespace rq
