/*
 * attn_capi.h - C ABI of the MI355X (gfx950) causal multi-head attention library
 * (libtcamd_attn.so).
 *
 * Every entry point takes plain device pointers, int sizes, a float scale and a
 * hipStream_t (an opaque pointer; pass NULL for the null stream).  Nothing here
 * allocates device memory or synchronises the host, and every entry point may be captured
 * into a HIP graph.  Work is enqueued on `stream`.
 *
 * State the library holds on the device (fixed arrays, never allocated per call):
 *   - the fp32 tiled kernels (attn_*_f32 forward and backward stages) pull tasks from
 *     counters in one of 64 slots per kernel family, taken in turn by each ordinary launch
 *     and left at zero when the launch ends; so at most 64 launches of one family may run
 *     at the same time (on different streams).  A launch captured into a graph takes no
 *     slot (it runs a static schedule), so replays of a graph, concurrent or not, share
 *     nothing.  The results do not depend on the schedule (bitwise);
 *   - attn_tiled_causal_backward_f32_noalloc keeps D in a scratch array shared by every
 *     call on the same GPU (see there).
 *
 * Every entry point returns an attn_status.  Arguments are validated on the host
 * before anything is launched: a non-zero status means nothing was enqueued (except
 * ATTN_ERROR_LAUNCH, which reports the HIP error of a launch that was attempted).
 *
 * Layouts (all row-major, contiguous):
 *   qkv, dqkv          (B, T, 3*H*d_head)       q | k | v column blocks, head h at [h*d, (h+1)*d)
 *   q, k, v, o, dO ... (B, H, T, d_head)        head-major
 *   m, l, D            (B, H, T)                per-row softmax statistics / dot(dO, O)
 *   scores, probs ...  (B*H*T, T)               materialised score matrices
 *
 * bf16 tensors are passed as attn_bf16 (the 16-bit pattern of a bfloat16 value).
 */
#ifndef TCAMD_ATTN_CAPI_H
#define TCAMD_ATTN_CAPI_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint16_t attn_bf16;

typedef enum attn_status {
    ATTN_SUCCESS = 0,
    ATTN_ERROR_INVALID_DIM = 1,          /* B, H, T or d_head <= 0, or a size that overflows */
    ATTN_ERROR_UNSUPPORTED_HEAD_DIM = 2, /* tiled kernels: d_head not in {32, 64, 128}        */
    ATTN_ERROR_NULL_POINTER = 3,         /* a required pointer is NULL                        */
    ATTN_ERROR_MISALIGNED = 4,           /* a pointer the kernel reads 16 bytes at a time is  */
                                         /* not 16-byte aligned                               */
    ATTN_ERROR_LAUNCH = 5,               /* hipGetLastError() after the launch was not success */
    ATTN_ERROR_INVALID_VALUE = 6,        /* scale not finite and > 0, batch count <= 0, ...   */
    ATTN_ERROR_SCRATCH_LIMIT = 7         /* no-alloc entry point: the problem needs more than */
                                         /* the library's fixed device scratch               */
} attn_status;

/* Human-readable name of a status code (static storage, never NULL). */
const char* attn_status_string(int status);

/* Library version: major*10000 + minor*100 + patch. */
int attn_version(void);

/* ------------------------------------------------------------------------------------------
 * QKV split-transpose  (B, T, 3*H*d) -> 3 x (B, H, T, d)  and its inverse scatter.
 * Any d_head >= 1; 16-byte vector path when d_head*sizeof(elem) is a multiple of 16 and
 * pointers are aligned, element path otherwise.
 * ------------------------------------------------------------------------------------------ */

/* Replaces qkv_split_transpose_forward, include/kernels/attention.cuh:5-11. */
int attn_qkv_split_transpose_forward_f32(const float* qkv, float* q, float* k, float* v,
                                         int B, int T, int H, int d_head, hipStream_t stream);
/* Replaces qkv_split_transpose_backward, include/kernels/attention.cuh:13-19. */
int attn_qkv_split_transpose_backward_f32(const float* dq, const float* dk, const float* dv,
                                          float* dqkv, int B, int T, int H, int d_head,
                                          hipStream_t stream);
/* bf16 fast path: no reference counterpart (the reference is fp32-only).  The f32->bf16
 * forward fuses the round-to-nearest-even cast into the copy; the bf16->f32 backward
 * widens exactly. */
int attn_qkv_split_transpose_forward_bf16(const attn_bf16* qkv, attn_bf16* q, attn_bf16* k,
                                          attn_bf16* v, int B, int T, int H, int d_head,
                                          hipStream_t stream);
int attn_qkv_split_transpose_forward_f32_bf16(const float* qkv, attn_bf16* q, attn_bf16* k,
                                              attn_bf16* v, int B, int T, int H, int d_head,
                                              hipStream_t stream);
int attn_qkv_split_transpose_backward_bf16(const attn_bf16* dq, const attn_bf16* dk,
                                           const attn_bf16* dv, attn_bf16* dqkv, int B, int T,
                                           int H, int d_head, hipStream_t stream);
int attn_qkv_split_transpose_backward_bf16_f32(const attn_bf16* dq, const attn_bf16* dk,
                                               const attn_bf16* dv, float* dqkv, int B, int T,
                                               int H, int d_head, hipStream_t stream);

/* ------------------------------------------------------------------------------------------
 * Head merge  (B, H, T, d) <-> (B, T, H*d)
 * ------------------------------------------------------------------------------------------ */

/* Replaces head_merge_transpose_forward, include/kernels/attention.cuh:91-97. */
int attn_head_merge_transpose_forward_f32(const float* in, float* out, int B, int H, int T,
                                          int d_head, hipStream_t stream);
/* Replaces head_merge_transpose_backward, include/kernels/attention.cuh:99-105. */
int attn_head_merge_transpose_backward_f32(const float* dout, float* din, int B, int H, int T,
                                           int d_head, hipStream_t stream);

/* ------------------------------------------------------------------------------------------
 * Materialised path: fused scaled causal softmax over (B*H*T, T) score rows.
 *   probs[r, j]   = exp(scale*s[r,j] - max_j'<=i scale*s[r,j']) / (sum + 1e-12)  for j <= i,
 *                   0 for j > i  (i = r mod T)
 *   dscores[r, j] = scale * p * (dp - sum_j'<=i dp*p)  for j <= i, else 0
 * ------------------------------------------------------------------------------------------ */

/* Replaces causal_softmax_forward, include/kernels/attention.cuh:21-31. */
int attn_causal_softmax_forward_f32(const float* scores, float* probs, int B, int H, int T,
                                    float scale, hipStream_t stream);
/* Replaces causal_softmax_backward, include/kernels/attention.cuh:80-89. */
int attn_causal_softmax_backward_f32(const float* dprobs, const float* probs, float* dscores,
                                     int B, int H, int T, float scale, hipStream_t stream);
/* No counterpart in the reference: the two softmax passes above with the zeros above the
 * diagonal written only up to the end of the zero_block-column block that holds the diagonal,
 * min(T, (i / zero_block + 1) * zero_block); the rest of each row is left as it was.  The
 * materialised attention entry points below run them with zero_block = 128, where their
 * products stop reading.  zero_block = 0 writes the whole suffix (as the functions above);
 * ATTN_ERROR_INVALID_VALUE unless zero_block is 0 or a positive multiple of 4. */
int attn_causal_softmax_forward_blocked_f32(const float* scores, float* probs, int B, int H,
                                            int T, float scale, int zero_block,
                                            hipStream_t stream);
int attn_causal_softmax_backward_blocked_f32(const float* dprobs, const float* probs,
                                             float* dscores, int B, int H, int T, float scale,
                                             int zero_block, hipStream_t stream);

/* ------------------------------------------------------------------------------------------
 * Materialised path: strided-batched fp32 GEMM (v_mfma_f32_32x32x2_f32) and the reference's
 * materialised attention sequences built from it and the softmax kernels above.
 * ------------------------------------------------------------------------------------------ */

/* Replaces matmul_batched_strided, include/kernels/matmul.cuh:44 (src/kernels/matmul.cu:167-207,
 * cublasSgemmStridedBatched).  Row-major, for b in [0, batch_count):
 *   C[b*strideC] (M x N, ldc = N) = alpha * op(A[b*strideA]) * op(B[b*strideB]) + beta * C
 * op(A) = A (M x K, lda = K) or, if transA, A^T of A stored K x M (lda = M); op(B) = B (K x N,
 * ldb = N) or, if transB, B^T of B stored N x K (ldb = K).  beta == 0 does not read C.
 * Strides >= 0; alpha, beta finite (else ATTN_ERROR_INVALID_VALUE).  No alignment needed. */
int attn_matmul_batched_strided_f32(const float* A, const float* B, float* C, int M, int N,
                                    int K, long long strideA, long long strideB,
                                    long long strideC, int batch_count, int transA, int transB,
                                    float alpha, float beta, hipStream_t stream);

/* The handle of the strided-batched GEMM: the counterpart of the cublasHandle_t that the
 * reference's matmul_batched_strided takes first (include/kernels/matmul.cuh:44-58, created at
 * src/model.cu:16-23).  The GEMM keeps no state, so the handle only records the device that
 * was current when it was created; a call through it while another device is current fails
 * with ATTN_ERROR_INVALID_VALUE before anything is launched.  Host memory only. */
typedef struct attn_gemm_context* attn_gemm_handle;
/* Create a handle bound to the current device (ATTN_ERROR_LAUNCH if there is none). */
int attn_gemm_create(attn_gemm_handle* handle);
/* Destroy a handle (NULL is accepted and ignored). */
int attn_gemm_destroy(attn_gemm_handle handle);
/* Device ordinal the handle is bound to, or -1 for a NULL handle. */
int attn_gemm_device(attn_gemm_handle handle);
/* No counterpart in the reference: attn_matmul_batched_strided_f32 (alpha 1, beta 0) for
 * operands with the structure of causal attention, which lets it skip work the causal mask
 * makes unused.  The materialised attention entry points below run their six products
 * through it.  `causal`:
 *   ATTN_GEMM_FULL       the full product (as attn_matmul_batched_strided_f32);
 *   ATTN_GEMM_LOWER_OUT  M == N; only C[i][j] with j <= i is needed (scores for a causal
 *                        softmax): 128 x 128 blocks of C wholly above the diagonal are not
 *                        written;
 *   ATTN_GEMM_LOWER_A    M == K; op(A)[i][k] == 0 for k > i (causal probabilities): those
 *                        terms are not computed;
 *   ATTN_GEMM_UPPER_A    M == K; op(A)[i][k] == 0 for k < i (their transpose): likewise.
 * The results equal the full product's for finite inputs (the skipped terms are exact
 * zeros; the skipped outputs are not written).  Other validation as the full product's;
 * ATTN_ERROR_INVALID_VALUE for an unknown `causal`, ATTN_ERROR_INVALID_DIM for M, N, K that
 * do not fit it. */
typedef enum attn_gemm_causal {
    ATTN_GEMM_FULL = 0,
    ATTN_GEMM_LOWER_OUT = 1,
    ATTN_GEMM_LOWER_A = 2,
    ATTN_GEMM_UPPER_A = 3
} attn_gemm_causal;
int attn_matmul_batched_strided_causal_f32(const float* A, const float* B, float* C, int M,
                                           int N, int K, long long strideA, long long strideB,
                                           long long strideC, int batch_count, int transA,
                                           int transB, int causal, hipStream_t stream);
/* Replaces matmul_batched_strided with its handle argument, include/kernels/matmul.cuh:44-58:
 * attn_matmul_batched_strided_f32 run through `handle` (ATTN_ERROR_NULL_POINTER if NULL). */
int attn_matmul_batched_strided_f32_h(attn_gemm_handle handle, const float* A, const float* B,
                                      float* C, int M, int N, int K, long long strideA,
                                      long long strideB, long long strideC, int batch_count,
                                      int transA, int transB, float alpha, float beta,
                                      hipStream_t stream);

/* The reference's materialised forward (src/model.cu:313-332), scores and probs (B*H*T, T):
 *   scores = Q K^T  ->  probs = causal_softmax_forward(scores, scale)  ->  out = probs V.
 * The contractions skip what the causal mask makes unused: scores is written where j <= i
 * (and in the rest of each 128 x 128 block that crosses the diagonal; blocks wholly above it
 * are left as they were, and the softmax never reads them), and out = probs V runs over
 * the nonzero part of probs only.  probs is written where j <= i and, as zeros, in the rest
 * of each 128 x 128 block that crosses the diagonal (the softmax with zero_block = 128); the
 * blocks wholly above the diagonal are left as they were, and nothing reads them.  out equals
 * the full product's for finite inputs. */
int attn_materialized_causal_forward_f32(const float* q, const float* k, const float* v,
                                         float* scores, float* probs, float* out, int B, int H,
                                         int T, int d_head, float scale, hipStream_t stream);

/* The reference's materialised backward (src/model.cu:617-650): dprobs = dO V^T,
 * dv = probs^T dO, dscores = causal_softmax_backward(dprobs, probs, scale), dq = dscores K,
 * dk = dscores^T Q.  dprobs and dscores are (B*H*T, T) scratch; dq, dk, dv are overwritten.
 * As in the forward, dprobs and dscores are written only in the 128 x 128 blocks at or
 * below the diagonal (dscores with zeros above the diagonal inside them), and the four
 * products with probs or dscores run over their nonzero parts. */
int attn_materialized_causal_backward_f32(const float* q, const float* k, const float* v,
                                          const float* probs, const float* dout, float* dprobs,
                                          float* dscores, float* dq, float* dk, float* dv,
                                          int B, int H, int T, int d_head, float scale,
                                          hipStream_t stream);

/* ------------------------------------------------------------------------------------------
 * Tiled (flash) causal attention, fp32 parity path: QK^T and PV on v_mfma_f32_32x32x2_f32.
 * d_head in {32, 64, 128}.  All (B,H,T,d) tensors and the stats must be 16-byte aligned.
 *
 * Forward writes out = softmax(mask(scale*Q K^T)) V and, when non-NULL,
 *   m_out[r] = max_j<=i scale*q_i.k_j,   l_out[r] = sum_j<=i exp(scale*q_i.k_j - m_out[r]),
 * so that P_ij = exp(scale*q_i.k_j - m_i) / l_i  (the contract of the reference stats).
 * ------------------------------------------------------------------------------------------ */

/* Replaces tiled_causal_attention_forward, include/kernels/attention.cuh:33-49. */
int attn_tiled_causal_forward_f32(const float* q, const float* k, const float* v, float* out,
                                  int B, int H, int T, int d_head, float scale, float* m_out,
                                  float* l_out, hipStream_t stream);

/* Replaces attention_precompute_dot_do_o, include/kernels/attention.cuh:51-58:
 * D[r] = sum_e dO[r,e] * O[r,e]. */
int attn_precompute_dot_do_o_f32(const float* dO, const float* O, float* D, int B, int H,
                                 int T, int d_head, hipStream_t stream);

/* Replaces tiled_causal_attention_backward, include/kernels/attention.cuh:60-78.
 * d_workspace holds B*H*T floats (it receives D).  m_ptr/l_ptr are the forward's stats.
 * dq, dk, dv are fully overwritten.  Enqueues the two stages below, in this order. */
int attn_tiled_causal_backward_f32(const float* q, const float* k, const float* v,
                                   const float* o, const float* do_ptr, const float* m_ptr,
                                   const float* l_ptr, float* dq, float* dk, float* dv,
                                   float* d_workspace, int B, int H, int T, int d_head,
                                   float scale, hipStream_t stream);

/* No counterpart in the reference.  For callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc): the same
 * backward as attn_tiled_causal_backward_f32, bitwise, without the caller's d_workspace.
 * D (B*H*T floats) goes to a fixed scratch array in device memory that the library holds on
 * each GPU it runs on until the process ends (ATTN_NOALLOC_SCRATCH_FLOATS floats, 16 MiB);
 * B*H*T above that fails with ATTN_ERROR_SCRATCH_LIMIT before anything is enqueued.  Nothing
 * is allocated.  Every call on one GPU shares that GPU's scratch, so calls that overlap in
 * time on one GPU (other streams, other host threads) race: serialise them. */
#define ATTN_NOALLOC_SCRATCH_FLOATS (1 << 22)
int attn_tiled_causal_backward_f32_noalloc(const float* q, const float* k, const float* v,
                                           const float* o, const float* do_ptr,
                                           const float* m_ptr, const float* l_ptr, float* dq,
                                           float* dk, float* dv, int B, int H, int T,
                                           int d_head, float scale, hipStream_t stream);

/* Stage 1 of attn_tiled_causal_backward_f32 (query-parallel): computes
 * D = rowsum(dO*O) into d_workspace and dq = scale * sum_j dS_ij k_j.
 * The reference splits the same work between attention.cu:659-692 and :696-812. */
int attn_tiled_causal_backward_dq_f32(const float* q, const float* k, const float* v,
                                      const float* o, const float* do_ptr, const float* m_ptr,
                                      const float* l_ptr, float* dq, float* d_workspace, int B,
                                      int H, int T, int d_head, float scale, hipStream_t stream);
/* Stage 2 (key-parallel): dk, dv from D in d_workspace (written by stage 1).
 * The reference computes the same in attention.cu:816-955. */
int attn_tiled_causal_backward_dkdv_f32(const float* q, const float* k, const float* v,
                                        const float* do_ptr, const float* m_ptr,
                                        const float* l_ptr, const float* d_workspace, float* dk,
                                        float* dv, int B, int H, int T, int d_head, float scale,
                                        hipStream_t stream);

/* ------------------------------------------------------------------------------------------
 * Tiled causal attention, bf16 fast path (no reference counterpart: the reference is
 * fp32-only).  bf16 Q/K/V/O/dO/dQ/dK/dV, fp32 statistics, fp32 accumulation on
 * v_mfma_f32_32x32x16_bf16.  Same stats contract P_ij = exp(scale*q_i.k_j - m_i) / l_i and
 * workspace size (B*H*T floats) as fp32, and the same log-sum-exp m + ln l, but m_out is the
 * forward's reference value rather than the row maximum: the maximum over the row's first 32
 * keys, raised to a later block's maximum only where the exponentials against it grow large
 * (a row sum of 2^16 over a 32-key block at d_head 32 and 64, an exponent above 8 at 128),
 * and l_out the sum against it.  The backward entry points take either form.
 * ------------------------------------------------------------------------------------------ */
int attn_tiled_causal_forward_bf16(const attn_bf16* q, const attn_bf16* k, const attn_bf16* v,
                                   attn_bf16* out, int B, int H, int T, int d_head, float scale,
                                   float* m_out, float* l_out, hipStream_t stream);
int attn_tiled_causal_backward_bf16(const attn_bf16* q, const attn_bf16* k,
                                    const attn_bf16* v, const attn_bf16* o,
                                    const attn_bf16* do_ptr, const float* m_ptr,
                                    const float* l_ptr, attn_bf16* dq, attn_bf16* dk,
                                    attn_bf16* dv, float* d_workspace, int B, int H, int T,
                                    int d_head, float scale, hipStream_t stream);
int attn_tiled_causal_backward_dq_bf16(const attn_bf16* q, const attn_bf16* k,
                                       const attn_bf16* v, const attn_bf16* o,
                                       const attn_bf16* do_ptr, const float* m_ptr,
                                       const float* l_ptr, attn_bf16* dq, float* d_workspace,
                                       int B, int H, int T, int d_head, float scale,
                                       hipStream_t stream);
int attn_tiled_causal_backward_dkdv_bf16(const attn_bf16* q, const attn_bf16* k,
                                         const attn_bf16* v, const attn_bf16* do_ptr,
                                         const float* m_ptr, const float* l_ptr,
                                         const float* d_workspace, attn_bf16* dk, attn_bf16* dv,
                                         int B, int H, int T, int d_head, float scale,
                                         hipStream_t stream);

/* ------------------------------------------------------------------------------------------
 * Packed QKV layout: attention straight from the QKV projection's output.
 * qkv (B, T, 3*H*d_head) as qkv_split_transpose_forward (include/kernels/attention.cuh:5-11)
 * reads it; dqkv (B, T, 3*H*d_head) as qkv_split_transpose_backward (:13-19) writes it.  The
 * split-transpose moves happen inside the attention kernels' tile copies and stores (no
 * head-major q/k/v/dq/dk/dv buffers).  Results are bitwise those of split-transpose + the
 * tiled entry points above.  out, o, dO stay head-major (B, H, T, d); stats and workspace as
 * above.  No counterpart in the reference: a fused form of its
 * split -> tiled_causal_attention_forward and tiled_causal_attention_backward -> split-back
 * sequence (src/model.cu:305-311, 609-653).
 * ------------------------------------------------------------------------------------------ */
int attn_packed_causal_forward_f32(const float* qkv, float* out, int B, int H, int T,
                                   int d_head, float scale, float* m_out, float* l_out,
                                   hipStream_t stream);
int attn_packed_causal_backward_f32(const float* qkv, const float* o, const float* do_ptr,
                                    const float* m_ptr, const float* l_ptr, float* dqkv,
                                    float* d_workspace, int B, int H, int T, int d_head,
                                    float scale, hipStream_t stream);
/* The two stages of the packed backward (enqueued in this order by the call above): stage 1
 * writes D into d_workspace and the q block of dqkv, stage 2 the k and v blocks. */
int attn_packed_causal_backward_dq_f32(const float* qkv, const float* o, const float* do_ptr,
                                       const float* m_ptr, const float* l_ptr, float* dqkv,
                                       float* d_workspace, int B, int H, int T, int d_head,
                                       float scale, hipStream_t stream);
int attn_packed_causal_backward_dkdv_f32(const float* qkv, const float* do_ptr,
                                         const float* m_ptr, const float* l_ptr,
                                         const float* d_workspace, float* dqkv, int B, int H,
                                         int T, int d_head, float scale, hipStream_t stream);
/* The packed / fused fp32 backward in the dS-first order (no counterpart in the reference):
 * prep writes D into d_workspace (the same sums as stage 1 above); dkdv_ds writes the k and
 * v blocks of dqkv and dS into ds_workspace; dq_ds writes the q block of dqkv as scale * dS K.
 * Stage 1 above computes S and dP again for dQ, two thirds of its fp32 MFMA work; here the
 * dK/dV stage hands them over as dS.  ds_workspace: attn_f32_ds_workspace_bytes(B, H, T,
 * d_head) bytes (B*H heads of n x n fp32, n = T rounded up to 32, held as 32 x 32 tiles in
 * a layout private to the two stages), 16-byte aligned; its contents need no initialisation.
 * That function returns 0 where the byte count exceeds SIZE_MAX, and the entry points reject
 * such shapes with ATTN_ERROR_INVALID_DIM.  D, dK and dV bitwise those of the two-stage
 * order, dQ within fp32 rounding of its. */
size_t attn_f32_ds_workspace_bytes(int B, int H, int T, int d_head);
/* 1 where a caller that chooses the order per shape should take the dS-first order: d_head
 * 32, 64 or 128 and ds_workspace at most 16 GiB (the same limit as the three-plane path's);
 * 0 elsewhere, where the two-stage entry points above need no T^2 workspace.  On the fp32
 * MFMA the dS-first backward measured 0.78-0.88x the two-stage time at d_head 32, 64 and 128
 * (T 1024 to 8192). */
int attn_f32_backward_uses_ds(int B, int H, int T, int d_head);
int attn_packed_causal_backward_ds_f32(const float* qkv, const float* o, const float* do_ptr,
                                       const float* m_ptr, const float* l_ptr, float* dqkv,
                                       float* d_workspace, float* ds_workspace, int B, int H,
                                       int T, int d_head, float scale, hipStream_t stream);
int attn_packed_causal_backward_prep_f32(const float* o, const float* do_ptr, float* d_workspace,
                                         int B, int H, int T, int d_head, hipStream_t stream);
int attn_packed_causal_backward_dkdv_ds_f32(const float* qkv, const float* do_ptr,
                                            const float* m_ptr, const float* l_ptr,
                                            const float* d_workspace, float* dqkv,
                                            float* ds_workspace, int B, int H, int T,
                                            int d_head, float scale, hipStream_t stream);
int attn_causal_backward_dq_ds_f32(const float* qkv, float* dqkv, const float* ds_workspace,
                                   int B, int H, int T, int d_head, float scale,
                                   hipStream_t stream);
int attn_packed_causal_forward_bf16(const attn_bf16* qkv, attn_bf16* out, int B, int H, int T,
                                    int d_head, float scale, float* m_out, float* l_out,
                                    hipStream_t stream);
int attn_packed_causal_backward_bf16(const attn_bf16* qkv, const attn_bf16* o,
                                     const attn_bf16* do_ptr, const float* m_ptr,
                                     const float* l_ptr, attn_bf16* dqkv, float* d_workspace,
                                     int B, int H, int T, int d_head, float scale,
                                     hipStream_t stream);
int attn_packed_causal_backward_dq_bf16(const attn_bf16* qkv, const attn_bf16* o,
                                        const attn_bf16* do_ptr, const float* m_ptr,
                                        const float* l_ptr, attn_bf16* dqkv, float* d_workspace,
                                        int B, int H, int T, int d_head, float scale,
                                        hipStream_t stream);
int attn_packed_causal_backward_dkdv_bf16(const attn_bf16* qkv, const attn_bf16* do_ptr,
                                          const float* m_ptr, const float* l_ptr,
                                          const float* d_workspace, attn_bf16* dqkv, int B,
                                          int H, int T, int d_head, float scale,
                                          hipStream_t stream);

/* ------------------------------------------------------------------------------------------
 * Fused layout: packed QKV in, merged heads out.  As the packed entry points above, but the
 * attention output `out` / `o` and its gradient `do_ptr` are in the (B, T, H*d_head) layout of
 * head_merge_transpose_forward's output (include/kernels/attention.cuh:91-105): one launch
 * replaces split-transpose -> tiled forward -> head merge, and the backward reads the
 * out-projection's input gradient directly (no head_merge_transpose_backward).  Results are
 * bitwise those of the packed entry points followed / preceded by the head merge.  No
 * counterpart in the reference: a fused form of its src/model.cu:305-336 and :602-653.
 * ------------------------------------------------------------------------------------------ */
int attn_fused_causal_forward_f32(const float* qkv, float* out, int B, int H, int T,
                                  int d_head, float scale, float* m_out, float* l_out,
                                  hipStream_t stream);
int attn_fused_causal_backward_f32(const float* qkv, const float* o, const float* do_ptr,
                                   const float* m_ptr, const float* l_ptr, float* dqkv,
                                   float* d_workspace, int B, int H, int T, int d_head,
                                   float scale, hipStream_t stream);
int attn_fused_causal_backward_dq_f32(const float* qkv, const float* o, const float* do_ptr,
                                      const float* m_ptr, const float* l_ptr, float* dqkv,
                                      float* d_workspace, int B, int H, int T, int d_head,
                                      float scale, hipStream_t stream);
int attn_fused_causal_backward_dkdv_f32(const float* qkv, const float* do_ptr,
                                        const float* m_ptr, const float* l_ptr,
                                        const float* d_workspace, float* dqkv, int B, int H,
                                        int T, int d_head, float scale, hipStream_t stream);
/* The dS-first order with the fused layout's o and dO (dq_ds above serves both layouts). */
int attn_fused_causal_backward_ds_f32(const float* qkv, const float* o, const float* do_ptr,
                                      const float* m_ptr, const float* l_ptr, float* dqkv,
                                      float* d_workspace, float* ds_workspace, int B, int H,
                                      int T, int d_head, float scale, hipStream_t stream);
int attn_fused_causal_backward_prep_f32(const float* o, const float* do_ptr, float* d_workspace,
                                        int B, int H, int T, int d_head, hipStream_t stream);
int attn_fused_causal_backward_dkdv_ds_f32(const float* qkv, const float* do_ptr,
                                           const float* m_ptr, const float* l_ptr,
                                           const float* d_workspace, float* dqkv,
                                           float* ds_workspace, int B, int H, int T, int d_head,
                                           float scale, hipStream_t stream);
int attn_fused_causal_forward_bf16(const attn_bf16* qkv, attn_bf16* out, int B, int H, int T,
                                   int d_head, float scale, float* m_out, float* l_out,
                                   hipStream_t stream);
int attn_fused_causal_backward_bf16(const attn_bf16* qkv, const attn_bf16* o,
                                    const attn_bf16* do_ptr, const float* m_ptr,
                                    const float* l_ptr, attn_bf16* dqkv, float* d_workspace,
                                    int B, int H, int T, int d_head, float scale,
                                    hipStream_t stream);
int attn_fused_causal_backward_dq_bf16(const attn_bf16* qkv, const attn_bf16* o,
                                       const attn_bf16* do_ptr, const float* m_ptr,
                                       const float* l_ptr, attn_bf16* dqkv, float* d_workspace,
                                       int B, int H, int T, int d_head, float scale,
                                       hipStream_t stream);
int attn_fused_causal_backward_dkdv_bf16(const attn_bf16* qkv, const attn_bf16* do_ptr,
                                         const float* m_ptr, const float* l_ptr,
                                         const float* d_workspace, attn_bf16* dqkv, int B,
                                         int H, int T, int d_head, float scale,
                                         hipStream_t stream);

/* ------------------------------------------------------------------------------------------
 * fp32 on bf16 matrix cores.  The fp32 entry points above run the fp32 MFMA (157 TFLOP/s
 * peak on MI355X); these compute the same fp32 attention on the bf16 MFMA (16x the rate):
 * every fp32 operand x is carried as three bf16 planes x_0 + x_1 + x_2 (24 significant
 * bits, all of fp32's) and every product a*b as the six plane products a_i*b_j, i + j <= 2
 * (what is left out is below 2^-23 |a*b|, about one fp32 rounding), accumulated in fp32.
 * Inputs, outputs and statistics are fp32 with the meaning of the packed / fused entry
 * points.  d_head 32 or 64.
 *
 * `planes` is caller-owned device memory of attn_f32x3_workspace_bytes(B, H, T, d_head)
 * bytes (16-byte aligned): the planes of q, k, v and dO (4 x 3 x B*H*T*d_head bf16), then,
 * where attn_f32x3_backward_uses_ds(B, H, T, d_head) is 1, dS: B*H x n x n fp32 with n = T
 * rounded up to 32, in 32 x 32 tiles (the one-call backward's dK/dV stage writes it for its
 * dQ stage).  The forward writes the planes of q, k and v; a backward with
 * kv_planes_ready = 1 reuses them (the caller guarantees that qkv and the workspace are
 * unchanged since that forward), with 0 it splits q, k and v again.  The backward's
 * d_workspace is the B*H*T floats of D, as in the other backward entry points.
 * No counterpart in the reference (an MI355X-specific form of
 * src/kernels/attention.cu:518-1012).
 * ------------------------------------------------------------------------------------------ */
size_t attn_f32x3_workspace_bytes(int B, int H, int T, int d_head);
/* The two parts of that workspace on their own: the planes (4 x 3 x B*H*T*d_head bf16) and
 * the dS area (0 where attn_f32x3_backward_uses_ds is 0).  attn_f32x3_workspace_bytes is
 * their sum.  A caller that keeps the planes of several layers alive between their forward
 * and backward (a training step) needs only one dS area: dS lives inside one backward call. */
size_t attn_f32x3_planes_bytes(int B, int H, int T, int d_head);
size_t attn_f32x3_ds_workspace_bytes(int B, int H, int T, int d_head);
/* 1 when the one-call backwards take the dS-first order (three stages: prep, dkdv_ds, dq_ds;
 * d_head 64 and dS at most 16 GiB), 0 when they take the two-stage order (dq, then dkdv).
 * The dS-first order saves the dQ stage's recomputation of S and dP for 8 bytes of HBM
 * traffic per stored dS element: faster at d_head 64, slower at 32. */
int attn_f32x3_backward_uses_ds(int B, int H, int T, int d_head);
int attn_packed_causal_forward_f32x3(const float* qkv, float* out, int B, int H, int T,
                                     int d_head, float scale, float* m_out, float* l_out,
                                     void* planes, hipStream_t stream);
int attn_fused_causal_forward_f32x3(const float* qkv, float* out, int B, int H, int T,
                                    int d_head, float scale, float* m_out, float* l_out,
                                    void* planes, hipStream_t stream);
int attn_packed_causal_backward_f32x3(const float* qkv, const float* o, const float* do_ptr,
                                      const float* m_ptr, const float* l_ptr, float* dqkv,
                                      float* d_workspace, int B, int H, int T, int d_head,
                                      float scale, void* planes, int kv_planes_ready,
                                      hipStream_t stream);
int attn_fused_causal_backward_f32x3(const float* qkv, const float* o, const float* do_ptr,
                                     const float* m_ptr, const float* l_ptr, float* dqkv,
                                     float* d_workspace, int B, int H, int T, int d_head,
                                     float scale, void* planes, int kv_planes_ready,
                                     hipStream_t stream);
/* The one-call backwards with dS in a separate buffer: `planes` of at least
 * attn_f32x3_planes_bytes, ds_workspace of attn_f32x3_ds_workspace_bytes (16-byte aligned,
 * no initialisation needed; NULL allowed where that size is 0, i.e. where the two-stage order
 * is taken).  Otherwise as attn_packed_causal_backward_f32x3 / attn_fused_causal_backward_f32x3,
 * with the same results bitwise. */
int attn_packed_causal_backward_ds_f32x3(const float* qkv, const float* o, const float* do_ptr,
                                         const float* m_ptr, const float* l_ptr, float* dqkv,
                                         float* d_workspace, float* ds_workspace, int B, int H,
                                         int T, int d_head, float scale, void* planes,
                                         int kv_planes_ready, hipStream_t stream);
int attn_fused_causal_backward_ds_f32x3(const float* qkv, const float* o, const float* do_ptr,
                                        const float* m_ptr, const float* l_ptr, float* dqkv,
                                        float* d_workspace, float* ds_workspace, int B, int H,
                                        int T, int d_head, float scale, void* planes,
                                        int kv_planes_ready, hipStream_t stream);
/* The three stages of the dS-first order, in order: prep writes the planes of dO (and of q,
 * k, v unless kv_planes_ready) and D; dkdv_ds (one function for both layouts: it reads dO
 * only through its planes) writes dK and dV into dqkv and dS into `planes`; dq_ds writes dQ
 * into dqkv from dS and the planes of k.  dkdv_ds and dq_ds return
 * ATTN_ERROR_UNSUPPORTED_HEAD_DIM (d_head other than 64) or ATTN_ERROR_INVALID_DIM (dS above
 * 16 GiB) where attn_f32x3_backward_uses_ds is 0: the workspace has no dS there. */
int attn_packed_causal_backward_prep_f32x3(const float* qkv, const float* o,
                                           const float* do_ptr, float* d_workspace, int B,
                                           int H, int T, int d_head, void* planes,
                                           int kv_planes_ready, hipStream_t stream);
int attn_fused_causal_backward_prep_f32x3(const float* qkv, const float* o, const float* do_ptr,
                                          float* d_workspace, int B, int H, int T, int d_head,
                                          void* planes, int kv_planes_ready,
                                          hipStream_t stream);
int attn_causal_backward_dkdv_ds_f32x3(const float* qkv, const float* m_ptr, const float* l_ptr,
                                       const float* d_workspace, float* dqkv, int B, int H,
                                       int T, int d_head, float scale, void* planes,
                                       hipStream_t stream);
int attn_causal_backward_dq_ds_f32x3(float* dqkv, int B, int H, int T, int d_head, float scale,
                                     const void* planes, hipStream_t stream);
/* The two-stage order, for every shape: stage 1 writes the planes of dO (and of q, k, v unless
 * kv_planes_ready), D and dQ, computing S and dP itself; stage 2 (one function for both
 * layouts) writes dK and dV from the planes in `planes`.  The same D, dK and dV as the three
 * stages, bitwise; dQ within fp32 rounding of theirs.  Does not use the workspace's dS. */
int attn_packed_causal_backward_dq_f32x3(const float* qkv, const float* o,
                                         const float* do_ptr, const float* m_ptr,
                                         const float* l_ptr, float* dqkv, float* d_workspace,
                                         int B, int H, int T, int d_head, float scale,
                                         void* planes, int kv_planes_ready,
                                         hipStream_t stream);
int attn_fused_causal_backward_dq_f32x3(const float* qkv, const float* o, const float* do_ptr,
                                        const float* m_ptr, const float* l_ptr, float* dqkv,
                                        float* d_workspace, int B, int H, int T, int d_head,
                                        float scale, void* planes, int kv_planes_ready,
                                        hipStream_t stream);
int attn_causal_backward_dkdv_f32x3(const float* qkv, const float* m_ptr, const float* l_ptr,
                                    const float* d_workspace, float* dqkv, int B, int H, int T,
                                    int d_head, float scale, const void* planes,
                                    hipStream_t stream);
/* The same path with the reference's tiled-launcher arguments: separate head-major q, k, v
 * (and o, dO, dq, dk, dv) (B, H, T, d_head) as in tiled_causal_attention_forward / _backward
 * (include/kernels/attention.cuh:39-49, 63-78), plus the plane workspace. */
int attn_tiled_causal_forward_f32x3(const float* q, const float* k, const float* v,
                                    float* out, int B, int H, int T, int d_head, float scale,
                                    float* m_out, float* l_out, void* planes,
                                    hipStream_t stream);
int attn_tiled_causal_backward_f32x3(const float* q, const float* k, const float* v,
                                     const float* o, const float* do_ptr, const float* m_ptr,
                                     const float* l_ptr, float* dq, float* dk, float* dv,
                                     float* d_workspace, int B, int H, int T, int d_head,
                                     float scale, void* planes, int kv_planes_ready,
                                     hipStream_t stream);
int attn_tiled_causal_backward_dq_f32x3(const float* q, const float* k, const float* v,
                                        const float* o, const float* do_ptr,
                                        const float* m_ptr, const float* l_ptr, float* dq,
                                        float* d_workspace, int B, int H, int T, int d_head,
                                        float scale, void* planes, int kv_planes_ready,
                                        hipStream_t stream);
int attn_tiled_causal_backward_dkdv_f32x3(const float* k, const float* v, const float* m_ptr,
                                          const float* l_ptr, const float* d_workspace,
                                          float* dk, float* dv, int B, int H, int T,
                                          int d_head, float scale, const void* planes,
                                          hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* TCAMD_ATTN_CAPI_H */
