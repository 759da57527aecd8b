// launch.hpp - internal launchers, one per kernel family.  The C ABI (capi.hip) validates
// arguments and then calls these; they assume valid arguments and only enqueue work.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "device_common.hpp"

namespace tcamd {

enum class ElemType { F32, BF16 };

// Row-major (B, T, S, H, d) <-> S head-major tensors (B, H, T, d).  S = 3 for the QKV
// split (heads[0..2] = q, k, v), S = 1 for the head merge.  to_heads selects the
// direction.  Element types may differ (the cast is fused into the copy).
struct HeadPtrs {
    void* p[3];
};
void launch_stripe_transpose(const void* src, ElemType src_t, void* dst, ElemType dst_t,
                             const HeadPtrs& heads, bool to_heads, int B, int T, int S, int H,
                             int d, hipStream_t stream);

void launch_causal_softmax_fwd_f32(const float* scores, float* probs, int64_t rows, int T,
                                   float scale, hipStream_t stream);
void launch_causal_softmax_bwd_f32(const float* dprobs, const float* probs, float* dscores,
                                   int64_t rows, int T, float scale, hipStream_t stream);

// Row-major strided-batched C = alpha*op(A)*op(B) + beta*C, C (M x N) with ldc = N.
void launch_batched_gemm_f32(const float* A, const float* B, float* C, int M, int N, int K,
                             long long sA, long long sB, long long sC, int batch, bool transA,
                             bool transB, float alpha, float beta, hipStream_t stream);

void launch_dot_do_o_f32(const float* dO, const float* O, float* D, int64_t rows, int d,
                         hipStream_t stream);

// The flash kernels address their operands through HeadViews: xv for q, k, v (head-major,
// or the packed QKV layout with q/k/v pointing at their column blocks), ov for o and dO
// (head-major), gv for dq, dk, dv (head-major or packed like xv).
void launch_flash_fwd_f32(const float* q, const float* k, const float* v, float* o,
                          float* m_out, float* l_out, int BH, int T, int d, float scale,
                          const HeadView& xv, const HeadView& ov, hipStream_t stream);
void launch_flash_bwd_dq_f32(const float* q, const float* k, const float* v, const float* o,
                             const float* dO, const float* m, const float* l, float* dq,
                             float* Dws, int BH, int T, int d, float scale, const HeadView& xv,
                             const HeadView& ov, const HeadView& gv, hipStream_t stream);
void launch_flash_bwd_dkdv_f32(const float* q, const float* k, const float* v,
                               const float* dO, const float* m, const float* l,
                               const float* Dws, float* dk, float* dv, int BH, int T, int d,
                               float scale, const HeadView& xv, const HeadView& ov,
                               const HeadView& gv, hipStream_t stream);

void launch_flash_fwd_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                           uint16_t* o, float* m_out, float* l_out, int BH, int T, int d,
                           float scale, const HeadView& xv, const HeadView& ov,
                           hipStream_t stream);
void launch_flash_bwd_dq_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                              const uint16_t* o, const uint16_t* dO, const float* m,
                              const float* l, uint16_t* dq, float* Dws, int BH, int T, int d,
                              float scale, const HeadView& xv, const HeadView& ov,
                              const HeadView& gv, hipStream_t stream);
void launch_flash_bwd_dkdv_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                const uint16_t* dO, const float* m, const float* l,
                                const float* Dws, uint16_t* dk, uint16_t* dv, int BH, int T,
                                int d, float scale, const HeadView& xv, const HeadView& ov,
                                const HeadView& gv, hipStream_t stream);

}  // namespace tcamd
