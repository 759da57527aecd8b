// kernels/matmul.h - the strided-batched GEMM of the materialised attention mode, MI355X build.
//
// Reference: include/kernels/matmul.cuh:44-58 (matmul_batched_strided, implemented at
// src/kernels/matmul.cu:167-207 with cublasSgemmStridedBatched), called at
// src/model.cu:314-332 and 618-650.  Same parameter list, order and defaults, row-major
// semantics.  The leading handle is this library's gemm_handle_t (create it once with
// gemm_create, as the reference's model creates its cuBLAS handle): the GEMM is a
// stateless HIP kernel, so the handle only pins the device it was created on.  Throws
// std::runtime_error on a non-zero status.
#pragma once

#include "kernels/attention.h"

using gemm_handle_t = attn_gemm_handle;

// Create / destroy a handle bound to the current device.
inline void gemm_create(gemm_handle_t* handle) {
    tcamd::check_status(attn_gemm_create(handle), "gemm_create");
}
inline void gemm_destroy(gemm_handle_t handle) {
    tcamd::check_status(attn_gemm_destroy(handle), "gemm_destroy");
}

// C[i] = alpha * (op_A(A[i]) * op_B(B[i])) + beta * C[i] for i < batch_count (row-major),
// the reference's declaration with its defaults.
inline void matmul_batched_strided(gemm_handle_t handle, const float* A, const float* B,
                                   float* C, int M, int N, int K, long long int strideA,
                                   long long int strideB, long long int strideC,
                                   int batch_count, bool transA = false, bool transB = false,
                                   float alpha = 1.0f, float beta = 0.0f,
                                   hipStream_t stream = nullptr) {
    tcamd::check_status(
        attn_matmul_batched_strided_f32_h(handle, A, B, C, M, N, K, strideA, strideB, strideC,
                                          batch_count, transA ? 1 : 0, transB ? 1 : 0, alpha,
                                          beta, stream),
        "matmul_batched_strided");
}

// The same without a handle (the GEMM needs none).
inline void matmul_batched_strided(const float* A, const float* B, float* C, int M, int N,
                                   int K, long long int strideA, long long int strideB,
                                   long long int strideC, int batch_count, bool transA = false,
                                   bool transB = false, float alpha = 1.0f, float beta = 0.0f,
                                   hipStream_t stream = nullptr) {
    tcamd::check_status(
        attn_matmul_batched_strided_f32(A, B, C, M, N, K, strideA, strideB, strideC,
                                        batch_count, transA ? 1 : 0, transB ? 1 : 0, alpha,
                                        beta, stream),
        "matmul_batched_strided");
}

// The reference's materialised attention forward (src/model.cu:313-332) and backward
// (src/model.cu:617-650) as single calls; scores/probs/dprobs/dscores are (B*H*T, T).
inline void materialized_causal_attention_forward(const float* q, const float* k,
                                                  const float* v, float* scores, float* probs,
                                                  float* out, int B, int H, int T, int d_head,
                                                  float scale, hipStream_t stream = nullptr) {
    tcamd::check_status(attn_materialized_causal_forward_f32(q, k, v, scores, probs, out, B, H,
                                                             T, d_head, scale, stream),
                        "materialized_causal_attention_forward");
}

inline void materialized_causal_attention_backward(const float* q, const float* k,
                                                   const float* v, const float* probs,
                                                   const float* dout, float* dprobs,
                                                   float* dscores, float* dq, float* dk,
                                                   float* dv, int B, int H, int T, int d_head,
                                                   float scale, hipStream_t stream = nullptr) {
    tcamd::check_status(
        attn_materialized_causal_backward_f32(q, k, v, probs, dout, dprobs, dscores, dq, dk, dv,
                                              B, H, T, d_head, scale, stream),
        "materialized_causal_attention_backward");
}
