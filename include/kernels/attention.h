// kernels/attention.h - C++ launchers of the causal attention hot path, MI355X build.
//
// Same names, parameter order and defaults as the reference's
// include/kernels/attention.cuh:5-105, with cudaStream_t replaced by hipStream_t.  Each
// launcher forwards to the C ABI in attn_capi.h and throws std::runtime_error on a
// non-zero status, the way the reference's callers wrap CUDA calls in CUDA_CHECK
// (include/common.h:10-20).  Unlike the reference, an unsupported d_head is an error,
// never a silent no-op (reference: src/kernels/attention.cu:651-655, 1009-1011).
//
// bf16 launchers are additions (the reference is fp32-only); they never overload the
// fp32 names.
#pragma once

#include <stdexcept>
#include <string>

#include "attn_capi.h"

namespace tcamd {
inline void check_status(int status, const char* what) {
    if (status != ATTN_SUCCESS) {
        throw std::runtime_error(std::string(what) + ": " + attn_status_string(status));
    }
}
}  // namespace tcamd

// Split & transpose QKV: (B, T, 3*H*d_head) -> 3 tensors of (B, H, T, d_head).
// Reference: include/kernels/attention.cuh:5-11.
inline void qkv_split_transpose_forward(const float* qkv, float* q, float* k, float* v, int B,
                                        int T, int H, int d_head, hipStream_t stream = nullptr) {
    tcamd::check_status(
        attn_qkv_split_transpose_forward_f32(qkv, q, k, v, B, T, H, d_head, stream),
        "qkv_split_transpose_forward");
}

// Reference: include/kernels/attention.cuh:13-19.
inline void qkv_split_transpose_backward(const float* dq, const float* dk, const float* dv,
                                         float* dqkv, int B, int T, int H, int d_head,
                                         hipStream_t stream = nullptr) {
    tcamd::check_status(
        attn_qkv_split_transpose_backward_f32(dq, dk, dv, dqkv, B, T, H, d_head, stream),
        "qkv_split_transpose_backward");
}

// probs[b,h,i,j] = softmax(scores[b,h,i,j] * scale) over j <= i, else 0.
// Reference: include/kernels/attention.cuh:21-31.
inline void causal_softmax_forward(const float* scores, float* probs, int B, int H, int T,
                                   float scale, hipStream_t stream = nullptr) {
    tcamd::check_status(attn_causal_softmax_forward_f32(scores, probs, B, H, T, scale, stream),
                        "causal_softmax_forward");
}

// Reference: include/kernels/attention.cuh:33-49.
inline void tiled_causal_attention_forward(const float* q, const float* k, const float* v,
                                           float* out, int B, int H, int T, int d_head,
                                           float scale, float* m_out = nullptr,
                                           float* l_out = nullptr,
                                           hipStream_t stream = nullptr) {
    tcamd::check_status(attn_tiled_causal_forward_f32(q, k, v, out, B, H, T, d_head, scale,
                                                      m_out, l_out, stream),
                        "tiled_causal_attention_forward");
}

// D_i = sum_d dO[i,d] * O[i,d].  Reference: include/kernels/attention.cuh:51-58.
inline void attention_precompute_dot_do_o(const float* dO, const float* O, float* D, int B,
                                          int H, int T, int d_head,
                                          hipStream_t stream = nullptr) {
    tcamd::check_status(attn_precompute_dot_do_o_f32(dO, O, D, B, H, T, d_head, stream),
                        "attention_precompute_dot_do_o");
}

// Reference: include/kernels/attention.cuh:60-78.  d_workspace: B*H*T floats.
inline void tiled_causal_attention_backward(const float* q, const float* k, const float* v,
                                            const float* o, const float* do_ptr,
                                            const float* m_ptr, const float* l_ptr, float* dq,
                                            float* dk, float* dv, float* d_workspace, int B,
                                            int H, int T, int d_head, float scale,
                                            hipStream_t stream = nullptr) {
    tcamd::check_status(
        attn_tiled_causal_backward_f32(q, k, v, o, do_ptr, m_ptr, l_ptr, dq, dk, dv,
                                       d_workspace, B, H, T, d_head, scale, stream),
        "tiled_causal_attention_backward");
}

// No counterpart in the reference: tiled_causal_attention_backward without d_workspace, for
// callers that cannot allocate (D lives in the library's fixed device scratch; B*H*T up to
// ATTN_NOALLOC_SCRATCH_FLOATS; calls that overlap in time on one GPU race).
inline void tiled_causal_attention_backward_noalloc(const float* q, const float* k,
                                                    const float* v, const float* o,
                                                    const float* do_ptr, const float* m_ptr,
                                                    const float* l_ptr, float* dq, float* dk,
                                                    float* dv, int B, int H, int T, int d_head,
                                                    float scale, hipStream_t stream = nullptr) {
    tcamd::check_status(
        attn_tiled_causal_backward_f32_noalloc(q, k, v, o, do_ptr, m_ptr, l_ptr, dq, dk, dv, B,
                                               H, T, d_head, scale, stream),
        "tiled_causal_attention_backward_noalloc");
}

// dscores = scale * probs * (dprobs - sum(dprobs * probs)) for j <= i, else 0.
// Reference: include/kernels/attention.cuh:80-89.
inline void causal_softmax_backward(const float* dprobs, const float* probs, float* dscores,
                                    int B, int H, int T, float scale,
                                    hipStream_t stream = nullptr) {
    tcamd::check_status(
        attn_causal_softmax_backward_f32(dprobs, probs, dscores, B, H, T, scale, stream),
        "causal_softmax_backward");
}

// (B, H, T, d_head) -> (B, T, H*d_head).  Reference: include/kernels/attention.cuh:91-97.
inline void head_merge_transpose_forward(const float* in, float* out, int B, int H, int T,
                                         int d_head, hipStream_t stream = nullptr) {
    tcamd::check_status(attn_head_merge_transpose_forward_f32(in, out, B, H, T, d_head, stream),
                        "head_merge_transpose_forward");
}

// (B, T, H*d_head) -> (B, H, T, d_head).  Reference: include/kernels/attention.cuh:99-105.
inline void head_merge_transpose_backward(const float* dout, float* din, int B, int H, int T,
                                          int d_head, hipStream_t stream = nullptr) {
    tcamd::check_status(
        attn_head_merge_transpose_backward_f32(dout, din, B, H, T, d_head, stream),
        "head_merge_transpose_backward");
}

// ---- bf16 fast path (additions; bf16 tensors as attn_bf16 bit patterns) ----------------

inline void qkv_split_transpose_forward_bf16(const attn_bf16* qkv, attn_bf16* q, attn_bf16* k,
                                             attn_bf16* v, int B, int T, int H, int d_head,
                                             hipStream_t stream = nullptr) {
    tcamd::check_status(
        attn_qkv_split_transpose_forward_bf16(qkv, q, k, v, B, T, H, d_head, stream),
        "qkv_split_transpose_forward_bf16");
}

inline void qkv_split_transpose_forward_f32_to_bf16(const float* qkv, attn_bf16* q,
                                                    attn_bf16* k, attn_bf16* v, int B, int T,
                                                    int H, int d_head,
                                                    hipStream_t stream = nullptr) {
    tcamd::check_status(
        attn_qkv_split_transpose_forward_f32_bf16(qkv, q, k, v, B, T, H, d_head, stream),
        "qkv_split_transpose_forward_f32_to_bf16");
}

inline void qkv_split_transpose_backward_bf16(const attn_bf16* dq, const attn_bf16* dk,
                                              const attn_bf16* dv, attn_bf16* dqkv, int B,
                                              int T, int H, int d_head,
                                              hipStream_t stream = nullptr) {
    tcamd::check_status(
        attn_qkv_split_transpose_backward_bf16(dq, dk, dv, dqkv, B, T, H, d_head, stream),
        "qkv_split_transpose_backward_bf16");
}

inline void qkv_split_transpose_backward_bf16_to_f32(const attn_bf16* dq, const attn_bf16* dk,
                                                     const attn_bf16* dv, float* dqkv, int B,
                                                     int T, int H, int d_head,
                                                     hipStream_t stream = nullptr) {
    tcamd::check_status(
        attn_qkv_split_transpose_backward_bf16_f32(dq, dk, dv, dqkv, B, T, H, d_head, stream),
        "qkv_split_transpose_backward_bf16_to_f32");
}

inline void tiled_causal_attention_forward_bf16(const attn_bf16* q, const attn_bf16* k,
                                                const attn_bf16* v, attn_bf16* out, int B,
                                                int H, int T, int d_head, float scale,
                                                float* m_out = nullptr, float* l_out = nullptr,
                                                hipStream_t stream = nullptr) {
    tcamd::check_status(attn_tiled_causal_forward_bf16(q, k, v, out, B, H, T, d_head, scale,
                                                       m_out, l_out, stream),
                        "tiled_causal_attention_forward_bf16");
}

inline void tiled_causal_attention_backward_bf16(
    const attn_bf16* q, const attn_bf16* k, const attn_bf16* v, const attn_bf16* o,
    const attn_bf16* do_ptr, const float* m_ptr, const float* l_ptr, attn_bf16* dq,
    attn_bf16* dk, attn_bf16* dv, float* d_workspace, int B, int H, int T, int d_head,
    float scale, hipStream_t stream = nullptr) {
    tcamd::check_status(
        attn_tiled_causal_backward_bf16(q, k, v, o, do_ptr, m_ptr, l_ptr, dq, dk, dv,
                                        d_workspace, B, H, T, d_head, scale, stream),
        "tiled_causal_attention_backward_bf16");
}

// ---- packed QKV layout (additions; no counterpart in the reference) -----------------------
// Attention straight from the QKV projection's output qkv (B, T, 3*H*d_head), with the
// gradient written straight into dqkv (B, T, 3*H*d_head): one launcher replaces
// qkv_split_transpose_forward + tiled_causal_attention_forward (src/model.cu:305-311), the
// other tiled_causal_attention_backward + qkv_split_transpose_backward (:609-615, 653).
// Results are bitwise those of the unfused sequences; out, o, dO stay (B, H, T, d_head).

inline void packed_causal_attention_forward(const float* qkv, float* out, int B, int H, int T,
                                            int d_head, float scale, float* m_out = nullptr,
                                            float* l_out = nullptr,
                                            hipStream_t stream = nullptr) {
    tcamd::check_status(
        attn_packed_causal_forward_f32(qkv, out, B, H, T, d_head, scale, m_out, l_out, stream),
        "packed_causal_attention_forward");
}

inline void packed_causal_attention_backward(const float* qkv, const float* o,
                                             const float* do_ptr, const float* m_ptr,
                                             const float* l_ptr, float* dqkv,
                                             float* d_workspace, int B, int H, int T,
                                             int d_head, float scale,
                                             hipStream_t stream = nullptr) {
    tcamd::check_status(attn_packed_causal_backward_f32(qkv, o, do_ptr, m_ptr, l_ptr, dqkv,
                                                        d_workspace, B, H, T, d_head, scale,
                                                        stream),
                        "packed_causal_attention_backward");
}

inline void packed_causal_attention_forward_bf16(const attn_bf16* qkv, attn_bf16* out, int B,
                                                 int H, int T, int d_head, float scale,
                                                 float* m_out = nullptr,
                                                 float* l_out = nullptr,
                                                 hipStream_t stream = nullptr) {
    tcamd::check_status(
        attn_packed_causal_forward_bf16(qkv, out, B, H, T, d_head, scale, m_out, l_out, stream),
        "packed_causal_attention_forward_bf16");
}

inline void packed_causal_attention_backward_bf16(const attn_bf16* qkv, const attn_bf16* o,
                                                  const attn_bf16* do_ptr, const float* m_ptr,
                                                  const float* l_ptr, attn_bf16* dqkv,
                                                  float* d_workspace, int B, int H, int T,
                                                  int d_head, float scale,
                                                  hipStream_t stream = nullptr) {
    tcamd::check_status(attn_packed_causal_backward_bf16(qkv, o, do_ptr, m_ptr, l_ptr, dqkv,
                                                         d_workspace, B, H, T, d_head, scale,
                                                         stream),
                        "packed_causal_attention_backward_bf16");
}

// ---- fused layout: packed QKV in, merged heads out (additions; no counterpart) ----------
// As the packed launchers, with the attention output and its gradient in the (B, T, H*d_head)
// layout of head_merge_transpose_forward's output: the forward also replaces the head merge
// at src/model.cu:336, the backward the head_merge_transpose_backward at :602.

inline void fused_causal_attention_forward(const float* qkv, float* out, int B, int H, int T,
                                           int d_head, float scale, float* m_out = nullptr,
                                           float* l_out = nullptr,
                                           hipStream_t stream = nullptr) {
    tcamd::check_status(
        attn_fused_causal_forward_f32(qkv, out, B, H, T, d_head, scale, m_out, l_out, stream),
        "fused_causal_attention_forward");
}

inline void fused_causal_attention_backward(const float* qkv, const float* o,
                                            const float* do_ptr, const float* m_ptr,
                                            const float* l_ptr, float* dqkv, float* d_workspace,
                                            int B, int H, int T, int d_head, float scale,
                                            hipStream_t stream = nullptr) {
    tcamd::check_status(attn_fused_causal_backward_f32(qkv, o, do_ptr, m_ptr, l_ptr, dqkv,
                                                       d_workspace, B, H, T, d_head, scale,
                                                       stream),
                        "fused_causal_attention_backward");
}

inline void fused_causal_attention_forward_bf16(const attn_bf16* qkv, attn_bf16* out, int B,
                                                int H, int T, int d_head, float scale,
                                                float* m_out = nullptr, float* l_out = nullptr,
                                                hipStream_t stream = nullptr) {
    tcamd::check_status(
        attn_fused_causal_forward_bf16(qkv, out, B, H, T, d_head, scale, m_out, l_out, stream),
        "fused_causal_attention_forward_bf16");
}

// The fp32 backward in the dS-first order: dK/dV write dS into ds_workspace
// (attn_f32_ds_workspace_bytes(B, H, T, d_head) bytes, caller-owned, shareable across calls
// on one stream), dQ is computed from it.  D, dK, dV bitwise those of the calls above, dQ
// within fp32 rounding.  No counterpart in the reference.
inline void packed_causal_attention_backward_ds_f32(const float* qkv, const float* o,
                                                    const float* do_ptr, const float* m_ptr,
                                                    const float* l_ptr, float* dqkv,
                                                    float* d_workspace, float* ds_workspace,
                                                    int B, int H, int T, int d_head,
                                                    float scale, hipStream_t stream = nullptr) {
    tcamd::check_status(attn_packed_causal_backward_ds_f32(qkv, o, do_ptr, m_ptr, l_ptr, dqkv,
                                                           d_workspace, ds_workspace, B, H, T,
                                                           d_head, scale, stream),
                        "packed_causal_attention_backward_ds_f32");
}
inline void fused_causal_attention_backward_ds_f32(const float* qkv, const float* o,
                                                   const float* do_ptr, const float* m_ptr,
                                                   const float* l_ptr, float* dqkv,
                                                   float* d_workspace, float* ds_workspace,
                                                   int B, int H, int T, int d_head, float scale,
                                                   hipStream_t stream = nullptr) {
    tcamd::check_status(attn_fused_causal_backward_ds_f32(qkv, o, do_ptr, m_ptr, l_ptr, dqkv,
                                                          d_workspace, ds_workspace, B, H, T,
                                                          d_head, scale, stream),
                        "fused_causal_attention_backward_ds_f32");
}

inline void fused_causal_attention_backward_bf16(const attn_bf16* qkv, const attn_bf16* o,
                                                 const attn_bf16* do_ptr, const float* m_ptr,
                                                 const float* l_ptr, attn_bf16* dqkv,
                                                 float* d_workspace, int B, int H, int T,
                                                 int d_head, float scale,
                                                 hipStream_t stream = nullptr) {
    tcamd::check_status(attn_fused_causal_backward_bf16(qkv, o, do_ptr, m_ptr, l_ptr, dqkv,
                                                        d_workspace, B, H, T, d_head, scale,
                                                        stream),
                        "fused_causal_attention_backward_bf16");
}

// fp32 on the bf16 matrix cores: the packed / fused launchers above with every fp32 operand
// carried as three bf16 planes in `planes` (attn_f32x3_workspace_bytes(B, H, T, d_head)
// bytes, caller-owned).  The backward reuses the planes of q, k and v the forward left there
// when kv_planes_ready is true.  No counterpart in the reference.
inline void packed_causal_attention_forward_f32x3(const float* qkv, float* out, int B, int H,
                                                  int T, int d_head, float scale, void* planes,
                                                  float* m_out = nullptr,
                                                  float* l_out = nullptr,
                                                  hipStream_t stream = nullptr) {
    tcamd::check_status(attn_packed_causal_forward_f32x3(qkv, out, B, H, T, d_head, scale,
                                                         m_out, l_out, planes, stream),
                        "packed_causal_attention_forward_f32x3");
}

inline void packed_causal_attention_backward_f32x3(const float* qkv, const float* o,
                                                   const float* do_ptr, const float* m_ptr,
                                                   const float* l_ptr, float* dqkv,
                                                   float* d_workspace, int B, int H, int T,
                                                   int d_head, float scale, void* planes,
                                                   bool kv_planes_ready = true,
                                                   hipStream_t stream = nullptr) {
    tcamd::check_status(attn_packed_causal_backward_f32x3(qkv, o, do_ptr, m_ptr, l_ptr, dqkv,
                                                          d_workspace, B, H, T, d_head, scale,
                                                          planes, kv_planes_ready ? 1 : 0,
                                                          stream),
                        "packed_causal_attention_backward_f32x3");
}

inline void fused_causal_attention_forward_f32x3(const float* qkv, float* out, int B, int H,
                                                 int T, int d_head, float scale, void* planes,
                                                 float* m_out = nullptr, float* l_out = nullptr,
                                                 hipStream_t stream = nullptr) {
    tcamd::check_status(attn_fused_causal_forward_f32x3(qkv, out, B, H, T, d_head, scale,
                                                        m_out, l_out, planes, stream),
                        "fused_causal_attention_forward_f32x3");
}

inline void fused_causal_attention_backward_f32x3(const float* qkv, const float* o,
                                                  const float* do_ptr, const float* m_ptr,
                                                  const float* l_ptr, float* dqkv,
                                                  float* d_workspace, int B, int H, int T,
                                                  int d_head, float scale, void* planes,
                                                  bool kv_planes_ready = true,
                                                  hipStream_t stream = nullptr) {
    tcamd::check_status(attn_fused_causal_backward_f32x3(qkv, o, do_ptr, m_ptr, l_ptr, dqkv,
                                                         d_workspace, B, H, T, d_head, scale,
                                                         planes, kv_planes_ready ? 1 : 0,
                                                         stream),
                        "fused_causal_attention_backward_f32x3");
}

// The same backwards with dS in its own buffer: `planes` of attn_f32x3_planes_bytes (kept
// per layer from the forward), `ds_workspace` of attn_f32x3_ds_workspace_bytes (one buffer
// may serve every layer: dS lives inside one call).  Results bitwise those above.
inline void packed_causal_attention_backward_ds_f32x3(
    const float* qkv, const float* o, const float* do_ptr, const float* m_ptr,
    const float* l_ptr, float* dqkv, float* d_workspace, float* ds_workspace, int B, int H,
    int T, int d_head, float scale, void* planes, bool kv_planes_ready = true,
    hipStream_t stream = nullptr) {
    tcamd::check_status(
        attn_packed_causal_backward_ds_f32x3(qkv, o, do_ptr, m_ptr, l_ptr, dqkv, d_workspace,
                                             ds_workspace, B, H, T, d_head, scale, planes,
                                             kv_planes_ready ? 1 : 0, stream),
        "packed_causal_attention_backward_ds_f32x3");
}

inline void fused_causal_attention_backward_ds_f32x3(
    const float* qkv, const float* o, const float* do_ptr, const float* m_ptr,
    const float* l_ptr, float* dqkv, float* d_workspace, float* ds_workspace, int B, int H,
    int T, int d_head, float scale, void* planes, bool kv_planes_ready = true,
    hipStream_t stream = nullptr) {
    tcamd::check_status(
        attn_fused_causal_backward_ds_f32x3(qkv, o, do_ptr, m_ptr, l_ptr, dqkv, d_workspace,
                                            ds_workspace, B, H, T, d_head, scale, planes,
                                            kv_planes_ready ? 1 : 0, stream),
        "fused_causal_attention_backward_ds_f32x3");
}

// The reference's tiled launchers (separate head-major tensors) for fp32 on the bf16 matrix
// cores; `planes` as above.
inline void tiled_causal_attention_forward_f32x3(const float* q, const float* k, const float* v,
                                                 float* out, int B, int H, int T, int d_head,
                                                 float scale, void* planes,
                                                 float* m_out = nullptr, float* l_out = nullptr,
                                                 hipStream_t stream = nullptr) {
    tcamd::check_status(attn_tiled_causal_forward_f32x3(q, k, v, out, B, H, T, d_head, scale,
                                                        m_out, l_out, planes, stream),
                        "tiled_causal_attention_forward_f32x3");
}

inline void tiled_causal_attention_backward_f32x3(const float* q, const float* k,
                                                  const float* v, const float* o,
                                                  const float* do_ptr, const float* m_ptr,
                                                  const float* l_ptr, float* dq, float* dk,
                                                  float* dv, float* d_workspace, int B, int H,
                                                  int T, int d_head, float scale, void* planes,
                                                  bool kv_planes_ready = true,
                                                  hipStream_t stream = nullptr) {
    tcamd::check_status(attn_tiled_causal_backward_f32x3(q, k, v, o, do_ptr, m_ptr, l_ptr, dq,
                                                         dk, dv, d_workspace, B, H, T, d_head,
                                                         scale, planes,
                                                         kv_planes_ready ? 1 : 0, stream),
                        "tiled_causal_attention_backward_f32x3");
}
