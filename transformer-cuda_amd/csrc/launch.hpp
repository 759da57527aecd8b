// launch.hpp - internal launchers, one per kernel family.  The C ABI (capi.hip) validates
// arguments and then calls these; they assume valid arguments and only enqueue work.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "device_common.hpp"

namespace tcamd {

// A launcher that found it could not launch (and enqueued nothing) records that here; the
// C ABI's status check reports it as ATTN_ERROR_LAUNCH and clears it.  Per host thread.
void note_launch_failure();
bool take_launch_failure();

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

// zero_block = 0: the masked suffix of every row is written as zeros (the reference's
// semantics); Z > 0: only up to the end of the Z-column block that holds the diagonal.
void launch_causal_softmax_fwd_f32(const float* scores, float* probs, int64_t rows, int T,
                                   float scale, hipStream_t stream, int zero_block = 0);
void launch_causal_softmax_bwd_f32(const float* dprobs, const float* probs, float* dscores,
                                   int64_t rows, int T, float scale, hipStream_t stream,
                                   int zero_block = 0);

// Causal structure a batched GEMM may exploit (the materialised attention's contractions;
// the public matmul_batched_strided always computes the full product):
//   kGemmFull     the full product;
//   kGemmLowerOut C is needed only at col <= row (S = QK^T, dP = dO V^T, read only by the
//                 causal softmax): output tiles wholly above the diagonal are not written;
//   kGemmLowerA   op(A)[m][k] = 0 for k > m (A = P or dS, whose upper triangle the softmax
//                 writes as zeros): the k loop of a tile stops after its last row;
//   kGemmUpperA   op(A)[m][k] = 0 for k < m (op(A) = P^T or dS^T): the k loop of a tile
//                 starts at its first row.
// Skipped terms are exact zeros, so for finite inputs the results equal the full product's.
// (The same values as attn_gemm_causal of the C ABI.)
enum GemmTri { kGemmFull = 0, kGemmLowerOut = 1, kGemmLowerA = 2, kGemmUpperA = 3 };

// Row-major strided-batched C = alpha*op(A)*op(B) + beta*C, C (M x N) with ldc = N.
void launch_batched_gemm_f32(const float* A, const float* B, float* C, int M, int N, int K,
                             long long sA, long long sB, long long sC, int batch, bool transA,
                             bool transB, float alpha, float beta, hipStream_t stream,
                             GemmTri tri = kGemmFull);

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
// Unless ds is null, dS is written as well (fp32, layout of launch_flash_bwd_dkdv_f32x3's),
// for launch_flash_bwd_dq_ds_f32.
void launch_flash_bwd_dkdv_f32(const float* q, const float* k, const float* v,
                               const float* dO, const float* m, const float* l,
                               const float* Dws, float* dk, float* dv, int BH, int T, int d,
                               float scale, const HeadView& xv, const HeadView& ov,
                               const HeadView& gv, hipStream_t stream, float* ds = nullptr);
// D = rowsum(dO o O) (views ov) into Dws, with the sums of launch_flash_bwd_dq_f32's D.
void launch_bwd_d_rows_f32(const float* dO, const float* O, const HeadView& ov, float* Dws,
                           int BH, int T, int d, hipStream_t stream);
// dQ = scale * dS K on the fp32 MFMA (k rows: view kv; dq: view gv).
void launch_flash_bwd_dq_ds_f32(const float* k, const HeadView& kv, const float* ds, float* dq,
                                const HeadView& gv, int BH, int T, int d, float scale,
                                hipStream_t stream);

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

// An fp32 (B*H, T, d) view (d % 8 == 0, rows 16-byte aligned) as three head-major bf16
// planes (hi, mid, lo) at dst, dst + pstride, dst + 2 pstride; ntens such tensors in one
// launch, tensor j from src + j*src_step to dst + j*dst_step.
void launch_split_planes(const float* src, const HeadView& sv, uint16_t* dst, size_t pstride,
                         int BH, int T, int d, hipStream_t stream, int ntens = 1,
                         size_t src_step = 0, size_t dst_step = 0);

// fp32 attention on bf16 MFMAs: every fp32 operand carried as three bf16 planes (hi, mid,
// lo; bf16_tile.hpp), products as six plane products.  Q is read in fp32 (view qv) and
// split in registers, its planes written to q_planes (laid out as k's) unless null; k and v
// point at plane 0 of planes pstride elements apart, each plane addressed by xv; O is fp32.
// d = 32 or 64.
void launch_flash_fwd_f32x3(const float* q, const HeadView& qv, const uint16_t* k,
                            const uint16_t* v, size_t pstride, uint16_t* q_planes, float* o,
                            float* m_out, float* l_out, int BH, int T, int d, float scale,
                            const HeadView& xv, const HeadView& ov, hipStream_t stream);
// Stage 1 (D and dQ): q, o, dO fp32 rows (views qv, ov), k and v plane tensors (view kv);
// dq fp32 (view gv); the planes of dO written to do_planes (laid out as k's) unless null.
void launch_flash_bwd_dq_f32x3(const float* q, const HeadView& qv, const uint16_t* k,
                               const uint16_t* v, const HeadView& kv, size_t pstride,
                               uint16_t* do_planes, const float* o, const float* dO,
                               const HeadView& ov,
                               const float* m, const float* l, float* dq, const HeadView& gv,
                               float* Dws, int BH, int T, int d, float scale,
                               hipStream_t stream);
// Stage 2 (dK, dV): q and dO plane tensors (view tv), k and v fp32 rows (view kv); dk, dv
// fp32 (view gv).  Unless ds is null, dS is written out as well (fp32, the tiles of ds_tile
// at or below the diagonal; keys >= T: zeros), for launch_flash_bwd_dq_ds_f32x3.
void launch_flash_bwd_dkdv_f32x3(const uint16_t* q, const uint16_t* dO, const HeadView& tv,
                                 size_t pstride, const float* k, const float* v,
                                 const HeadView& kv, const float* m, const float* l,
                                 const float* Dws, float* dk, float* dv, const HeadView& gv,
                                 int BH, int T, int d, float scale, hipStream_t stream,
                                 float* ds = nullptr);
// The side of a head's square dS: T rounded up to 32.
constexpr int ds_rows(int T) { return (T + 31) / 32 * 32; }
// The dS area of the dS-first backwards: B*H heads of n x n fp32 (n = ds_rows(T)), each as
// (n/32) x (n/32) tiles of 32 queries x 32 keys; tile (qt, kt) of head bh is 4 KB contiguous
// from element ds_tile(bh, n, qt, kt), rows (queries) of 128 bytes.  The dK/dV stage writes
// the tiles with kt <= qt and the dQ stage reads them, each tile as one contiguous block.
constexpr size_t ds_tile(int bh, int n, int qt, int kt) {
    return ((static_cast<size_t>(bh) * (n / 32) + qt) * (n / 32) + kt) * 1024;
}
// Before stage 2 when stage 1 comes after it: D = rowsum(dO o O) into Dws (the same
// operations as stage 1's) and the planes of dO (laid out as k's, view kv).
void launch_bwd_prep_f32x3(const float* o, const float* dO, const HeadView& ov,
                           uint16_t* do_planes, const HeadView& kv, size_t pstride, float* Dws,
                           int BH, int T, int d, hipStream_t stream);
// Stage 1 from the dS of stage 2: dQ = scale * dS K (k plane tensors, view kv; dq fp32,
// view gv).
void launch_flash_bwd_dq_ds_f32x3(const uint16_t* k, const HeadView& kv, size_t pstride,
                                  const float* ds, float* dq, const HeadView& gv, int BH, int T,
                                  int d, float scale, hipStream_t stream);

}  // namespace tcamd
