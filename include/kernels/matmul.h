// kernels/matmul.h - the strided-batched GEMM of the materialised attention mode, MI355X build.
//
// Reference: include/kernels/matmul.cuh:44 (matmul_batched_strided, implemented at
// src/kernels/matmul.cu:167-207 with cublasSgemmStridedBatched).  Same parameters and
// row-major semantics minus the cuBLAS handle: the library's GEMM is a stateless HIP kernel,
// so there is no handle to create, bind to a stream or destroy.  Throws std::runtime_error
// on a non-zero status.
#pragma once

#include "kernels/attention.h"

// C_b (M x N) = alpha * op(A_b) * op(B_b) + beta * C_b for b < batch_count (row-major).
inline void matmul_batched_strided(const float* A, const float* B, float* C, int M, int N,
                                   int K, long long int strideA, long long int strideB,
                                   long long int strideC, int batch_count, bool transA,
                                   bool transB, float alpha, float beta,
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
