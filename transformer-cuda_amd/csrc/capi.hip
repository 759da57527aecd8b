// capi.hip - the extern "C" boundary (include/attn_capi.h).
//
// Each entry point validates its arguments on the host and returns a status before any
// HIP call, so the validation is testable on a machine without a GPU.  Only then does it
// enqueue the kernels and report the launch status.  Nothing here allocates or
// synchronises.
#include <math.h>
#include <stdint.h>

#include <atomic>

#include "../../include/attn_capi.h"
#include "launch.hpp"

namespace tcamd {
namespace {
thread_local bool t_launch_failed = false;
}  // namespace
void note_launch_failure() { t_launch_failed = true; }
bool take_launch_failure() {
    const bool f = t_launch_failed;
    t_launch_failed = false;
    return f;
}
}  // namespace tcamd

namespace {

using tcamd::ElemType;
using tcamd::HeadPtrs;

constexpr int64_t kInt32Max = 2147483647;

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_dims4(int B, int H, int T, int d) {
    if (B <= 0 || H <= 0 || T <= 0 || d <= 0) return ATTN_ERROR_INVALID_DIM;
    // Kernels index within one head in 32-bit and count (b, h) pairs in 32-bit.
    if (static_cast<int64_t>(T) * d > kInt32Max) return ATTN_ERROR_INVALID_DIM;
    if (static_cast<int64_t>(B) * H > 65535LL * 1024) return ATTN_ERROR_INVALID_DIM;
    return ATTN_SUCCESS;
}

int check_tiled(int B, int H, int T, int d, float scale) {
    const int st = check_dims4(B, H, T, d);
    if (st != ATTN_SUCCESS) return st;
    if (d != 32 && d != 64 && d != 128) return ATTN_ERROR_UNSUPPORTED_HEAD_DIM;
    if (!(scale > 0.0f) || !isfinite(scale)) return ATTN_ERROR_INVALID_VALUE;
    // grid = B*H * ceil(T / 128) workgroups
    const int64_t tiles = (static_cast<int64_t>(T) + 127) / 128;
    if (static_cast<int64_t>(B) * H * tiles > kInt32Max) return ATTN_ERROR_INVALID_DIM;
    return ATTN_SUCCESS;
}

int check_split(const void* a, const void* b, const void* c, const void* dd, int B, int T,
                int H, int d) {
    if (a == nullptr || b == nullptr || c == nullptr || dd == nullptr)
        return ATTN_ERROR_NULL_POINTER;
    const int st = check_dims4(B, H, T, d);
    if (st != ATTN_SUCCESS) return st;
    if (static_cast<int64_t>(B) * H > 65535) return ATTN_ERROR_INVALID_DIM;  // grid.y
    return ATTN_SUCCESS;
}

int check_materialized(int B, int H, int T, int d, float scale) {
    const int st = check_dims4(B, H, T, d);
    if (st != ATTN_SUCCESS) return st;
    if (!(scale > 0.0f) || !isfinite(scale)) return ATTN_ERROR_INVALID_VALUE;
    const int64_t tiles = ((static_cast<int64_t>(T) + 63) / 64) * ((static_cast<int64_t>(T) + 63) / 64);
    if (tiles * B * H > kInt32Max) return ATTN_ERROR_INVALID_DIM;
    return ATTN_SUCCESS;
}

int launch_status() {
    const hipError_t e = hipGetLastError();
    const bool failed = tcamd::take_launch_failure();
    return e == hipSuccess && !failed ? ATTN_SUCCESS : ATTN_ERROR_LAUNCH;
}

void clear_error() {
    (void)hipGetLastError();
    (void)tcamd::take_launch_failure();
}

int split_common(const void* rm, ElemType rm_t, void* q, void* k, void* v, ElemType h_t,
                 bool to_heads, int B, int T, int H, int d, hipStream_t stream) {
    const int st = check_split(rm, q, k, v, B, T, H, d);
    if (st != ATTN_SUCCESS) return st;
    HeadPtrs heads{{q, k, v}};
    clear_error();
    if (to_heads) {
        tcamd::launch_stripe_transpose(rm, rm_t, nullptr, h_t, heads, true, B, T, 3, H, d,
                                       stream);
    } else {
        tcamd::launch_stripe_transpose(nullptr, h_t, const_cast<void*>(rm), rm_t, heads, false,
                                       B, T, 3, H, d, stream);
    }
    return launch_status();
}

// ---- packed-QKV implementations (shared by the packed and fused entry points) ----------
// q, k, v are read from qkv (B, T, 3C) and dq, dk, dv written into dqkv; o and dO are
// head-major (B, H, T, d) or, `merged`, in the (B, T, C) layout of the head merge.

void flash_fwd(const float* q, const float* k, const float* v, float* o, float* m, float* l,
               int BH, int T, int d, float scale, const tcamd::HeadView& xv,
               const tcamd::HeadView& ov, hipStream_t s) {
    tcamd::launch_flash_fwd_f32(q, k, v, o, m, l, BH, T, d, scale, xv, ov, s);
}
void flash_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o, float* m,
               float* l, int BH, int T, int d, float scale, const tcamd::HeadView& xv,
               const tcamd::HeadView& ov, hipStream_t s) {
    tcamd::launch_flash_fwd_bf16(q, k, v, o, m, l, BH, T, d, scale, xv, ov, s);
}
void flash_dq(const float* q, const float* k, const float* v, const float* o, const float* dO,
              const float* m, const float* l, float* dq, float* ws, int BH, int T, int d,
              float scale, const tcamd::HeadView& xv, const tcamd::HeadView& ov,
              const tcamd::HeadView& gv, hipStream_t s) {
    tcamd::launch_flash_bwd_dq_f32(q, k, v, o, dO, m, l, dq, ws, BH, T, d, scale, xv, ov, gv, s);
}
void flash_dq(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* o,
              const uint16_t* dO, const float* m, const float* l, uint16_t* dq, float* ws,
              int BH, int T, int d, float scale, const tcamd::HeadView& xv,
              const tcamd::HeadView& ov, const tcamd::HeadView& gv, hipStream_t s) {
    tcamd::launch_flash_bwd_dq_bf16(q, k, v, o, dO, m, l, dq, ws, BH, T, d, scale, xv, ov, gv, s);
}
void flash_dkdv(const float* q, const float* k, const float* v, const float* dO, const float* m,
                const float* l, const float* ws, float* dk, float* dv, int BH, int T, int d,
                float scale, const tcamd::HeadView& xv, const tcamd::HeadView& ov,
                const tcamd::HeadView& gv, hipStream_t s) {
    tcamd::launch_flash_bwd_dkdv_f32(q, k, v, dO, m, l, ws, dk, dv, BH, T, d, scale, xv, ov, gv,
                                     s);
}
void flash_dkdv(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* dO,
                const float* m, const float* l, const float* ws, uint16_t* dk, uint16_t* dv,
                int BH, int T, int d, float scale, const tcamd::HeadView& xv,
                const tcamd::HeadView& ov, const tcamd::HeadView& gv, hipStream_t s) {
    tcamd::launch_flash_bwd_dkdv_bf16(q, k, v, dO, m, l, ws, dk, dv, BH, T, d, scale, xv, ov, gv,
                                      s);
}

tcamd::HeadView out_view(int H, int T, int d, bool merged) {
    return merged ? tcamd::merged_view(H, T, d) : tcamd::head_major_view(H, T, d);
}

// The qkv row stride 3*H*d is an int in the kernels.
int check_packed(int B, int H, int T, int d, float scale) {
    const int st = check_tiled(B, H, T, d, scale);
    if (st != ATTN_SUCCESS) return st;
    if (3LL * H * d > kInt32Max) return ATTN_ERROR_INVALID_DIM;
    return ATTN_SUCCESS;
}

template <typename E>
int packed_forward(const E* qkv, E* out, int B, int H, int T, int d, float scale, float* m_out,
                   float* l_out, bool merged, hipStream_t stream) {
    if (qkv == nullptr || out == nullptr) return ATTN_ERROR_NULL_POINTER;
    const int st = check_packed(B, H, T, d, scale);
    if (st != ATTN_SUCCESS) return st;
    if (!aligned16(qkv) || !aligned16(out)) return ATTN_ERROR_MISALIGNED;
    const size_t C = static_cast<size_t>(H) * d;
    clear_error();
    flash_fwd(qkv, qkv + C, qkv + 2 * C, out, m_out, l_out, B * H, T, d, scale,
              tcamd::packed_qkv_view(H, T, d), out_view(H, T, d, merged), stream);
    return launch_status();
}

// Shared checks of the packed-layout backward stages.
int check_packed_bwd(const void* qkv, const void* dO, const void* m, const void* l,
                     const void* dqkv, const void* ws, int B, int H, int T, int d,
                     float scale) {
    if (qkv == nullptr || dO == nullptr || m == nullptr || l == nullptr || dqkv == nullptr ||
        ws == nullptr)
        return ATTN_ERROR_NULL_POINTER;
    const int st = check_packed(B, H, T, d, scale);
    if (st != ATTN_SUCCESS) return st;
    if (!aligned16(qkv) || !aligned16(dO) || !aligned16(dqkv)) return ATTN_ERROR_MISALIGNED;
    return ATTN_SUCCESS;
}

template <typename E>
int packed_backward_dq(const E* qkv, const E* o, const E* dO, const float* m, const float* l,
                       E* dqkv, float* ws, int B, int H, int T, int d, float scale, bool merged,
                       hipStream_t stream) {
    if (o == nullptr) return ATTN_ERROR_NULL_POINTER;
    const int st = check_packed_bwd(qkv, dO, m, l, dqkv, ws, B, H, T, d, scale);
    if (st != ATTN_SUCCESS) return st;
    if (!aligned16(o)) return ATTN_ERROR_MISALIGNED;
    const size_t C = static_cast<size_t>(H) * d;
    const tcamd::HeadView xv = tcamd::packed_qkv_view(H, T, d);
    clear_error();
    flash_dq(qkv, qkv + C, qkv + 2 * C, o, dO, m, l, dqkv, ws, B * H, T, d, scale, xv,
             out_view(H, T, d, merged), xv, stream);
    return launch_status();
}

template <typename E>
int packed_backward_dkdv(const E* qkv, const E* dO, const float* m, const float* l,
                         const float* ws, E* dqkv, int B, int H, int T, int d, float scale,
                         bool merged, hipStream_t stream) {
    const int st = check_packed_bwd(qkv, dO, m, l, dqkv, ws, B, H, T, d, scale);
    if (st != ATTN_SUCCESS) return st;
    const size_t C = static_cast<size_t>(H) * d;
    const tcamd::HeadView xv = tcamd::packed_qkv_view(H, T, d);
    clear_error();
    flash_dkdv(qkv, qkv + C, qkv + 2 * C, dO, m, l, ws, dqkv + C, dqkv + 2 * C, B * H, T, d,
               scale, xv, out_view(H, T, d, merged), xv, stream);
    return launch_status();
}

// ---- fp32 MFMA backward in the dS-first order: D; dK/dV writing dS into a caller
// workspace (B*H heads of n x n fp32, n = T rounded up to 32); dQ = scale * dS K.

// Elements of the dS area, or 0 when its byte count does not fit in size_t (shapes the
// dimension checks accept reach 4 * 2^12 * 2^52 bytes).
size_t ds_f32_elems(int B, int H, int T) {
    const size_t n = static_cast<size_t>(tcamd::ds_rows(T));  // <= 2^26: n*n fits
    const size_t bh = static_cast<size_t>(B) * H;
    if (bh > (SIZE_MAX / sizeof(float)) / (n * n)) return 0;
    return bh * n * n;
}

int packed_backward_prep_f32(const float* o, const float* dO, float* ws, int B, int H, int T,
                             int d, bool merged, hipStream_t stream) {
    if (o == nullptr || dO == nullptr || ws == nullptr) return ATTN_ERROR_NULL_POINTER;
    const int st = check_packed(B, H, T, d, 1.0f);
    if (st != ATTN_SUCCESS) return st;
    if (!aligned16(o) || !aligned16(dO)) return ATTN_ERROR_MISALIGNED;
    clear_error();
    tcamd::launch_bwd_d_rows_f32(dO, o, out_view(H, T, d, merged), ws, B * H, T, d, stream);
    return launch_status();
}

int packed_backward_dkdv_ds_f32(const float* qkv, const float* dO, const float* m,
                                const float* l, const float* ws, float* dqkv, float* ds, int B,
                                int H, int T, int d, float scale, bool merged,
                                hipStream_t stream) {
    if (ds == nullptr) return ATTN_ERROR_NULL_POINTER;
    const int st = check_packed_bwd(qkv, dO, m, l, dqkv, ws, B, H, T, d, scale);
    if (st != ATTN_SUCCESS) return st;
    if (ds_f32_elems(B, H, T) == 0) return ATTN_ERROR_INVALID_DIM;
    if (!aligned16(ds)) return ATTN_ERROR_MISALIGNED;
    const size_t C = static_cast<size_t>(H) * d;
    const tcamd::HeadView xv = tcamd::packed_qkv_view(H, T, d);
    clear_error();
    tcamd::launch_flash_bwd_dkdv_f32(qkv, qkv + C, qkv + 2 * C, dO, m, l, ws, dqkv + C,
                                     dqkv + 2 * C, B * H, T, d, scale, xv,
                                     out_view(H, T, d, merged), xv, stream, ds);
    return launch_status();
}

int backward_dq_ds_f32(const float* qkv, float* dqkv, const float* ds, int B, int H, int T,
                       int d, float scale, hipStream_t stream) {
    if (qkv == nullptr || dqkv == nullptr || ds == nullptr) return ATTN_ERROR_NULL_POINTER;
    const int st = check_packed(B, H, T, d, scale);
    if (st != ATTN_SUCCESS) return st;
    if (ds_f32_elems(B, H, T) == 0) return ATTN_ERROR_INVALID_DIM;
    if (!aligned16(qkv) || !aligned16(dqkv) || !aligned16(ds)) return ATTN_ERROR_MISALIGNED;
    const size_t C = static_cast<size_t>(H) * d;
    const tcamd::HeadView xv = tcamd::packed_qkv_view(H, T, d);
    clear_error();
    tcamd::launch_flash_bwd_dq_ds_f32(qkv + C, xv, ds, dqkv, xv, B * H, T, d, scale, stream);
    return launch_status();
}

int packed_backward_ds_f32(const float* qkv, const float* o, const float* dO, const float* m,
                           const float* l, float* dqkv, float* ws, float* ds, int B, int H,
                           int T, int d, float scale, bool merged, hipStream_t stream) {
    if (o == nullptr || ds == nullptr) return ATTN_ERROR_NULL_POINTER;
    int st = check_packed_bwd(qkv, dO, m, l, dqkv, ws, B, H, T, d, scale);
    if (st != ATTN_SUCCESS) return st;
    if (ds_f32_elems(B, H, T) == 0) return ATTN_ERROR_INVALID_DIM;     // before any launch
    if (!aligned16(o) || !aligned16(ds)) return ATTN_ERROR_MISALIGNED;  // before any launch
    st = packed_backward_prep_f32(o, dO, ws, B, H, T, d, merged, stream);
    if (st != ATTN_SUCCESS) return st;
    st = packed_backward_dkdv_ds_f32(qkv, dO, m, l, ws, dqkv, ds, B, H, T, d, scale, merged,
                                     stream);
    if (st != ATTN_SUCCESS) return st;
    return backward_dq_ds_f32(qkv, dqkv, ds, B, H, T, d, scale, stream);
}

template <typename E>
int packed_backward(const E* qkv, const E* o, const E* dO, const float* m, const float* l,
                    E* dqkv, float* ws, int B, int H, int T, int d, float scale, bool merged,
                    hipStream_t stream) {
    const int st = packed_backward_dq(qkv, o, dO, m, l, dqkv, ws, B, H, T, d, scale, merged,
                                      stream);
    if (st != ATTN_SUCCESS) return st;
    return packed_backward_dkdv(qkv, dO, m, l, ws, dqkv, B, H, T, d, scale, merged, stream);
}

// ---- fp32 on bf16 MFMAs: operands as three bf16 planes in a caller workspace -------------
// Workspace: four tensors (q, k, v, dO) x three planes x N = B*H*T*d bf16, head-major; then,
// when the one-call backward takes the dS-first order (uses_ds), dS: B*H x n x n fp32 with
// n = T rounded up to 32 (its dK/dV stage writes it, its dQ stage reads it).

constexpr int kPlaneTensors = 4;
constexpr int kPlanes = 3;

size_t plane_elems(int B, int H, int T, int d) {
    return static_cast<size_t>(B) * H * T * d;
}
uint16_t* plane_tensor(void* planes, size_t N, int tensor) {
    return static_cast<uint16_t*>(planes) + static_cast<size_t>(tensor) * kPlanes * N;
}
size_t ds_elems(int B, int H, int T) {
    const size_t n = static_cast<size_t>(tcamd::ds_rows(T));
    return static_cast<size_t>(B) * H * n * n;
}
float* ds_area(void* planes, size_t N) {
    return reinterpret_cast<float*>(plane_tensor(planes, N, kPlaneTensors));
}
// The dS area of a combined workspace (attn_f32x3_workspace_bytes): after the planes.
float* combined_ds(void* planes, int B, int H, int T, int d) {
    return planes == nullptr ? nullptr : ds_area(planes, plane_elems(B, H, T, d));
}

// The one-call backward's order.  dS-first (dK/dV writing dS, then dQ = dS K) saves the dQ
// stage's S and dP products, 48 of its 74 MFMAs per tile at d = 64, for 8 bytes of HBM
// traffic per stored element; measured faster at d = 64 (0.86-0.93x from T = 512 to 8192)
// and slower at d = 32 (1.02-1.22x), where the products saved are half as many.  dS takes
// 4 B*H*n^2 bytes of workspace: above kDsMaxBytes the two-stage order is taken instead.
constexpr size_t kDsMaxBytes = static_cast<size_t>(1) << 34;  // 16 GiB
bool uses_ds(int B, int H, int T, int d) {
    if (d != 64 || B <= 0 || H <= 0 || T <= 0) return false;
    const double n = static_cast<double>(tcamd::ds_rows(T));
    return 4.0 * B * H * n * n <= static_cast<double>(kDsMaxBytes);
}
int check_uses_ds(int B, int H, int T, int d) {
    if (uses_ds(B, H, T, d)) return ATTN_SUCCESS;
    return d != 64 ? ATTN_ERROR_UNSUPPORTED_HEAD_DIM : ATTN_ERROR_INVALID_DIM;
}

int check_f32x3(int B, int H, int T, int d, float scale) {
    const int st = check_packed(B, H, T, d, scale);
    if (st != ATTN_SUCCESS) return st;
    if (d != 32 && d != 64) return ATTN_ERROR_UNSUPPORTED_HEAD_DIM;
    return ATTN_SUCCESS;
}

// k and v of qkv (B, T, 3C) into their planes (tensors 1 and 2 of the workspace), one
// launch.
void split_kv_planes(const float* qkv, void* planes, int B, int H, int T, int d,
                     hipStream_t stream) {
    const size_t N = plane_elems(B, H, T, d), C = static_cast<size_t>(H) * d;
    tcamd::launch_split_planes(qkv + C, tcamd::packed_qkv_view(H, T, d),
                               plane_tensor(planes, N, 1), N, B * H, T, d, stream, 2, C,
                               kPlanes * N);
}

int packed_forward_f32x3(const float* qkv, float* out, int B, int H, int T, int d, float scale,
                         float* m_out, float* l_out, void* planes, bool merged,
                         hipStream_t stream) {
    if (qkv == nullptr || out == nullptr || planes == nullptr) return ATTN_ERROR_NULL_POINTER;
    const int st = check_f32x3(B, H, T, d, scale);
    if (st != ATTN_SUCCESS) return st;
    if (!aligned16(qkv) || !aligned16(out) || !aligned16(planes)) return ATTN_ERROR_MISALIGNED;
    const size_t N = plane_elems(B, H, T, d);
    clear_error();
    split_kv_planes(qkv, planes, B, H, T, d, stream);
    tcamd::launch_flash_fwd_f32x3(qkv, tcamd::packed_qkv_view(H, T, d),
                                  plane_tensor(planes, N, 1), plane_tensor(planes, N, 2), N,
                                  plane_tensor(planes, N, 0), out, m_out, l_out, B * H, T, d,
                                  scale, tcamd::head_major_view(H, T, d),
                                  out_view(H, T, d, merged), stream);
    return launch_status();
}

// Stage 1: the planes of q, k, v unless the forward's are ready; D and dQ, writing the
// planes of dO.
int packed_backward_dq_f32x3(const float* qkv, const float* o, const float* dO, const float* m,
                             const float* l, float* dqkv, float* ws, int B, int H, int T, int d,
                             float scale, void* planes, int kv_ready, bool merged,
                             hipStream_t stream) {
    if (o == nullptr || planes == nullptr) return ATTN_ERROR_NULL_POINTER;
    int st = check_packed_bwd(qkv, dO, m, l, dqkv, ws, B, H, T, d, scale);
    if (st != ATTN_SUCCESS) return st;
    st = check_f32x3(B, H, T, d, scale);
    if (st != ATTN_SUCCESS) return st;
    if (!aligned16(o) || !aligned16(planes)) return ATTN_ERROR_MISALIGNED;
    const size_t N = plane_elems(B, H, T, d);
    const tcamd::HeadView xv = tcamd::packed_qkv_view(H, T, d);
    const tcamd::HeadView ov = out_view(H, T, d, merged);
    clear_error();
    if (!kv_ready)  // q, k, v in one launch
        tcamd::launch_split_planes(qkv, xv, plane_tensor(planes, N, 0), N, B * H, T, d, stream,
                                   3, static_cast<size_t>(H) * d, kPlanes * N);
    tcamd::launch_flash_bwd_dq_f32x3(qkv, xv, plane_tensor(planes, N, 1),
                                     plane_tensor(planes, N, 2), tcamd::head_major_view(H, T, d),
                                     N, plane_tensor(planes, N, 3), o, dO, ov, m, l, dqkv, xv, ws,
                                     B * H, T, d, scale, stream);
    return launch_status();
}

// Stage 2: dK and dV from the planes of q and dO that stage 1 wrote.
int packed_backward_dkdv_f32x3(const float* qkv, const float* m, const float* l,
                               const float* ws, float* dqkv, int B, int H, int T, int d,
                               float scale, const void* planes, hipStream_t stream) {
    if (qkv == nullptr || m == nullptr || l == nullptr || ws == nullptr || dqkv == nullptr ||
        planes == nullptr)
        return ATTN_ERROR_NULL_POINTER;
    const int st = check_f32x3(B, H, T, d, scale);
    if (st != ATTN_SUCCESS) return st;
    if (!aligned16(qkv) || !aligned16(dqkv) || !aligned16(planes)) return ATTN_ERROR_MISALIGNED;
    const size_t N = plane_elems(B, H, T, d), C = static_cast<size_t>(H) * d;
    const tcamd::HeadView xv = tcamd::packed_qkv_view(H, T, d);
    void* pl = const_cast<void*>(planes);
    clear_error();
    tcamd::launch_flash_bwd_dkdv_f32x3(plane_tensor(pl, N, 0), plane_tensor(pl, N, 3),
                                       tcamd::head_major_view(H, T, d), N, qkv + C, qkv + 2 * C,
                                       xv, m, l, ws, dqkv + C, dqkv + 2 * C, xv, B * H, T, d,
                                       scale, stream);
    return launch_status();
}

// The one-call backward runs three stages: (1) the planes of q, k, v unless the forward's
// are ready, D and the planes of dO; (2) dK and dV, writing dS; (3) dQ from dS and k's
// planes.  dS carries the products of S and dP from (2) to (3), which would otherwise compute
// them again.
int packed_backward_prep_f32x3(const float* qkv, const float* o, const float* dO, float* ws,
                               int B, int H, int T, int d, void* planes, int kv_ready,
                               bool merged, hipStream_t stream) {
    if (qkv == nullptr || o == nullptr || dO == nullptr || ws == nullptr || planes == nullptr)
        return ATTN_ERROR_NULL_POINTER;
    const int st = check_f32x3(B, H, T, d, 1.0f);
    if (st != ATTN_SUCCESS) return st;
    if (!aligned16(qkv) || !aligned16(o) || !aligned16(dO) || !aligned16(planes))
        return ATTN_ERROR_MISALIGNED;
    const size_t N = plane_elems(B, H, T, d);
    clear_error();
    if (!kv_ready)  // q, k, v in one launch
        tcamd::launch_split_planes(qkv, tcamd::packed_qkv_view(H, T, d), plane_tensor(planes, N, 0),
                                   N, B * H, T, d, stream, 3, static_cast<size_t>(H) * d,
                                   kPlanes * N);
    tcamd::launch_bwd_prep_f32x3(o, dO, out_view(H, T, d, merged), plane_tensor(planes, N, 3),
                                 tcamd::head_major_view(H, T, d), N, ws, B * H, T, d, stream);
    return launch_status();
}

// ds: the dS area (ds_elems fp32, 16-byte aligned): after the planes in a workspace of
// attn_f32x3_workspace_bytes, or a separate buffer of attn_f32x3_ds_workspace_bytes.
int packed_backward_dkdv_ds_f32x3(const float* qkv, const float* m, const float* l,
                                  const float* ws, float* dqkv, int B, int H, int T, int d,
                                  float scale, void* planes, float* ds, hipStream_t stream) {
    if (qkv == nullptr || m == nullptr || l == nullptr || ws == nullptr || dqkv == nullptr ||
        planes == nullptr || ds == nullptr)
        return ATTN_ERROR_NULL_POINTER;
    int st = check_f32x3(B, H, T, d, scale);
    if (st != ATTN_SUCCESS) return st;
    st = check_uses_ds(B, H, T, d);
    if (st != ATTN_SUCCESS) return st;
    if (!aligned16(qkv) || !aligned16(dqkv) || !aligned16(planes) || !aligned16(ds))
        return ATTN_ERROR_MISALIGNED;
    const size_t N = plane_elems(B, H, T, d), C = static_cast<size_t>(H) * d;
    const tcamd::HeadView xv = tcamd::packed_qkv_view(H, T, d);
    clear_error();
    tcamd::launch_flash_bwd_dkdv_f32x3(plane_tensor(planes, N, 0), plane_tensor(planes, N, 3),
                                       tcamd::head_major_view(H, T, d), N, qkv + C, qkv + 2 * C,
                                       xv, m, l, ws, dqkv + C, dqkv + 2 * C, xv, B * H, T, d,
                                       scale, stream, ds);
    return launch_status();
}

int packed_backward_dq_ds_f32x3(float* dqkv, int B, int H, int T, int d, float scale,
                                const void* planes, const float* ds, hipStream_t stream) {
    if (dqkv == nullptr || planes == nullptr || ds == nullptr) return ATTN_ERROR_NULL_POINTER;
    int st = check_f32x3(B, H, T, d, scale);
    if (st != ATTN_SUCCESS) return st;
    st = check_uses_ds(B, H, T, d);
    if (st != ATTN_SUCCESS) return st;
    if (!aligned16(dqkv) || !aligned16(planes) || !aligned16(ds)) return ATTN_ERROR_MISALIGNED;
    const size_t N = plane_elems(B, H, T, d);
    void* pl = const_cast<void*>(planes);
    clear_error();
    tcamd::launch_flash_bwd_dq_ds_f32x3(plane_tensor(pl, N, 1), tcamd::head_major_view(H, T, d),
                                        N, ds, dqkv, tcamd::packed_qkv_view(H, T, d), B * H, T,
                                        d, scale, stream);
    return launch_status();
}

// ds: the dS area where uses_ds (ignored, and may be null, elsewhere).
int packed_backward_f32x3(const float* qkv, const float* o, const float* dO, const float* m,
                          const float* l, float* dqkv, float* ws, int B, int H, int T, int d,
                          float scale, void* planes, float* ds, int kv_ready, bool merged,
                          hipStream_t stream) {
    if (o == nullptr || planes == nullptr) return ATTN_ERROR_NULL_POINTER;
    int st = check_packed_bwd(qkv, dO, m, l, dqkv, ws, B, H, T, d, scale);
    if (st != ATTN_SUCCESS) return st;
    if (!uses_ds(B, H, T, d)) {  // the two-stage order
        st = packed_backward_dq_f32x3(qkv, o, dO, m, l, dqkv, ws, B, H, T, d, scale, planes,
                                      kv_ready, merged, stream);
        if (st != ATTN_SUCCESS) return st;
        return packed_backward_dkdv_f32x3(qkv, m, l, ws, dqkv, B, H, T, d, scale, planes,
                                          stream);
    }
    if (ds == nullptr) return ATTN_ERROR_NULL_POINTER;                  // before any launch
    if (!aligned16(ds) || !aligned16(planes)) return ATTN_ERROR_MISALIGNED;  // before any launch
    st = packed_backward_prep_f32x3(qkv, o, dO, ws, B, H, T, d, planes, kv_ready, merged, stream);
    if (st != ATTN_SUCCESS) return st;
    st = packed_backward_dkdv_ds_f32x3(qkv, m, l, ws, dqkv, B, H, T, d, scale, planes, ds,
                                       stream);
    if (st != ATTN_SUCCESS) return st;
    return packed_backward_dq_ds_f32x3(dqkv, B, H, T, d, scale, planes, ds, stream);
}

// ---- the same path from separate head-major q, k, v (the reference's tiled launchers) ----

int check_tiled_f32x3(int B, int H, int T, int d, float scale, const void* planes) {
    if (planes == nullptr) return ATTN_ERROR_NULL_POINTER;
    const int st = check_f32x3(B, H, T, d, scale);
    if (st != ATTN_SUCCESS) return st;
    return aligned16(planes) ? ATTN_SUCCESS : ATTN_ERROR_MISALIGNED;
}

int tiled_forward_f32x3(const float* q, const float* k, const float* v, float* out, int B, int H,
                        int T, int d, float scale, float* m_out, float* l_out, void* planes,
                        hipStream_t stream) {
    if (q == nullptr || k == nullptr || v == nullptr || out == nullptr)
        return ATTN_ERROR_NULL_POINTER;
    const int st = check_tiled_f32x3(B, H, T, d, scale, planes);
    if (st != ATTN_SUCCESS) return st;
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out))
        return ATTN_ERROR_MISALIGNED;
    const size_t N = plane_elems(B, H, T, d);
    const tcamd::HeadView hv = tcamd::head_major_view(H, T, d);
    clear_error();
    tcamd::launch_split_planes(k, hv, plane_tensor(planes, N, 1), N, B * H, T, d, stream);
    tcamd::launch_split_planes(v, hv, plane_tensor(planes, N, 2), N, B * H, T, d, stream);
    tcamd::launch_flash_fwd_f32x3(q, hv, plane_tensor(planes, N, 1), plane_tensor(planes, N, 2),
                                  N, plane_tensor(planes, N, 0), out, m_out, l_out, B * H, T, d,
                                  scale, hv, hv, stream);
    return launch_status();
}

int tiled_backward_dq_f32x3(const float* q, const float* k, const float* v, const float* o,
                            const float* dO, const float* m, const float* l, float* dq,
                            float* ws, int B, int H, int T, int d, float scale, void* planes,
                            int kv_ready, hipStream_t stream) {
    if (q == nullptr || k == nullptr || v == nullptr || o == nullptr || dO == nullptr ||
        m == nullptr || l == nullptr || dq == nullptr || ws == nullptr)
        return ATTN_ERROR_NULL_POINTER;
    const int st = check_tiled_f32x3(B, H, T, d, scale, planes);
    if (st != ATTN_SUCCESS) return st;
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o) || !aligned16(dO) ||
        !aligned16(dq))
        return ATTN_ERROR_MISALIGNED;
    const size_t N = plane_elems(B, H, T, d);
    const tcamd::HeadView hv = tcamd::head_major_view(H, T, d);
    clear_error();
    if (!kv_ready) {
        tcamd::launch_split_planes(q, hv, plane_tensor(planes, N, 0), N, B * H, T, d, stream);
        tcamd::launch_split_planes(k, hv, plane_tensor(planes, N, 1), N, B * H, T, d, stream);
        tcamd::launch_split_planes(v, hv, plane_tensor(planes, N, 2), N, B * H, T, d, stream);
    }
    tcamd::launch_flash_bwd_dq_f32x3(q, hv, plane_tensor(planes, N, 1),
                                     plane_tensor(planes, N, 2), hv, N,
                                     plane_tensor(planes, N, 3), o, dO, hv, m, l, dq, hv, ws,
                                     B * H, T, d, scale, stream);
    return launch_status();
}

int tiled_backward_dkdv_f32x3(const float* k, const float* v, const float* m, const float* l,
                              const float* ws, float* dk, float* dv, int B, int H, int T, int d,
                              float scale, const void* planes, hipStream_t stream) {
    if (k == nullptr || v == nullptr || m == nullptr || l == nullptr || ws == nullptr ||
        dk == nullptr || dv == nullptr)
        return ATTN_ERROR_NULL_POINTER;
    const int st = check_tiled_f32x3(B, H, T, d, scale, planes);
    if (st != ATTN_SUCCESS) return st;
    if (!aligned16(k) || !aligned16(v) || !aligned16(dk) || !aligned16(dv))
        return ATTN_ERROR_MISALIGNED;
    const size_t N = plane_elems(B, H, T, d);
    const tcamd::HeadView hv = tcamd::head_major_view(H, T, d);
    void* pl = const_cast<void*>(planes);
    clear_error();
    tcamd::launch_flash_bwd_dkdv_f32x3(plane_tensor(pl, N, 0), plane_tensor(pl, N, 3), hv, N, k,
                                       v, hv, m, l, ws, dk, dv, hv, B * H, T, d, scale, stream);
    return launch_status();
}

// The full backward in the order packed_backward_f32x3 takes.
int tiled_backward_f32x3(const float* q, const float* k, const float* v, const float* o,
                         const float* dO, const float* m, const float* l, float* dq, float* dk,
                         float* dv, float* ws, int B, int H, int T, int d, float scale,
                         void* planes, int kv_ready, hipStream_t stream) {
    if (!uses_ds(B, H, T, d)) {  // the two-stage order
        const int st = tiled_backward_dq_f32x3(q, k, v, o, dO, m, l, dq, ws, B, H, T, d, scale,
                                               planes, kv_ready, stream);
        if (st != ATTN_SUCCESS) return st;
        return tiled_backward_dkdv_f32x3(k, v, m, l, ws, dk, dv, B, H, T, d, scale, planes,
                                         stream);
    }
    if (q == nullptr || k == nullptr || v == nullptr || o == nullptr || dO == nullptr ||
        m == nullptr || l == nullptr || dq == nullptr || dk == nullptr || dv == nullptr ||
        ws == nullptr)
        return ATTN_ERROR_NULL_POINTER;
    const int st = check_tiled_f32x3(B, H, T, d, scale, planes);
    if (st != ATTN_SUCCESS) return st;
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o) || !aligned16(dO) ||
        !aligned16(dq) || !aligned16(dk) || !aligned16(dv))
        return ATTN_ERROR_MISALIGNED;
    const size_t N = plane_elems(B, H, T, d);
    const tcamd::HeadView hv = tcamd::head_major_view(H, T, d);
    float* ds = ds_area(planes, N);
    clear_error();
    if (!kv_ready) {
        tcamd::launch_split_planes(q, hv, plane_tensor(planes, N, 0), N, B * H, T, d, stream);
        tcamd::launch_split_planes(k, hv, plane_tensor(planes, N, 1), N, B * H, T, d, stream);
        tcamd::launch_split_planes(v, hv, plane_tensor(planes, N, 2), N, B * H, T, d, stream);
    }
    tcamd::launch_bwd_prep_f32x3(o, dO, hv, plane_tensor(planes, N, 3), hv, N, ws, B * H, T, d,
                                 stream);
    tcamd::launch_flash_bwd_dkdv_f32x3(plane_tensor(planes, N, 0), plane_tensor(planes, N, 3), hv,
                                       N, k, v, hv, m, l, ws, dk, dv, hv, B * H, T, d, scale,
                                       stream, ds);
    tcamd::launch_flash_bwd_dq_ds_f32x3(plane_tensor(planes, N, 1), hv, N, ds, dq, hv, B * H, T,
                                        d, scale, stream);
    return launch_status();
}

}  // namespace


extern "C" {

const char* attn_status_string(int status) {
    switch (status) {
        case ATTN_SUCCESS: return "success";
        case ATTN_ERROR_INVALID_DIM: return "invalid dimension (B, H, T, d_head or a size)";
        case ATTN_ERROR_UNSUPPORTED_HEAD_DIM: return "unsupported d_head (tiled kernels: 32, 64, 128)";
        case ATTN_ERROR_NULL_POINTER: return "required pointer is NULL";
        case ATTN_ERROR_MISALIGNED: return "pointer not 16-byte aligned";
        case ATTN_ERROR_LAUNCH: return "kernel launch failed";
        case ATTN_ERROR_INVALID_VALUE: return "invalid value (scale, alpha/beta, batch count or stride)";
        case ATTN_ERROR_SCRATCH_LIMIT: return "problem exceeds the fixed scratch of a no-alloc entry point";
        default: return "unknown status";
    }
}

int attn_version(void) { return 100; }

// ---- split-transpose --------------------------------------------------------------------

int attn_qkv_split_transpose_forward_f32(const float* qkv, float* q, float* k, float* v,
                                         int B, int T, int H, int d_head, hipStream_t stream) {
    return split_common(qkv, ElemType::F32, q, k, v, ElemType::F32, true, B, T, H, d_head,
                        stream);
}

int attn_qkv_split_transpose_backward_f32(const float* dq, const float* dk, const float* dv,
                                          float* dqkv, int B, int T, int H, int d_head,
                                          hipStream_t stream) {
    return split_common(dqkv, ElemType::F32, const_cast<float*>(dq), const_cast<float*>(dk),
                        const_cast<float*>(dv), ElemType::F32, false, B, T, H, d_head, stream);
}

int attn_qkv_split_transpose_forward_bf16(const attn_bf16* qkv, attn_bf16* q, attn_bf16* k,
                                          attn_bf16* v, int B, int T, int H, int d_head,
                                          hipStream_t stream) {
    return split_common(qkv, ElemType::BF16, q, k, v, ElemType::BF16, true, B, T, H, d_head,
                        stream);
}

int attn_qkv_split_transpose_forward_f32_bf16(const float* qkv, attn_bf16* q, attn_bf16* k,
                                              attn_bf16* v, int B, int T, int H, int d_head,
                                              hipStream_t stream) {
    return split_common(qkv, ElemType::F32, q, k, v, ElemType::BF16, true, B, T, H, d_head,
                        stream);
}

int attn_qkv_split_transpose_backward_bf16(const attn_bf16* dq, const attn_bf16* dk,
                                           const attn_bf16* dv, attn_bf16* dqkv, int B, int T,
                                           int H, int d_head, hipStream_t stream) {
    return split_common(dqkv, ElemType::BF16, const_cast<attn_bf16*>(dq),
                        const_cast<attn_bf16*>(dk), const_cast<attn_bf16*>(dv), ElemType::BF16,
                        false, B, T, H, d_head, stream);
}

int attn_qkv_split_transpose_backward_bf16_f32(const attn_bf16* dq, const attn_bf16* dk,
                                               const attn_bf16* dv, float* dqkv, int B, int T,
                                               int H, int d_head, hipStream_t stream) {
    return split_common(dqkv, ElemType::F32, const_cast<attn_bf16*>(dq),
                        const_cast<attn_bf16*>(dk), const_cast<attn_bf16*>(dv), ElemType::BF16,
                        false, B, T, H, d_head, stream);
}

// ---- head merge -------------------------------------------------------------------------

int attn_head_merge_transpose_forward_f32(const float* in, float* out, int B, int H, int T,
                                          int d_head, hipStream_t stream) {
    const int st = check_split(in, out, out, out, B, T, H, d_head);
    if (st != ATTN_SUCCESS) return st;
    HeadPtrs heads{{const_cast<float*>(in), nullptr, nullptr}};
    clear_error();
    tcamd::launch_stripe_transpose(nullptr, ElemType::F32, out, ElemType::F32, heads, false, B,
                                   T, 1, H, d_head, stream);
    return launch_status();
}

int attn_head_merge_transpose_backward_f32(const float* dout, float* din, int B, int H, int T,
                                           int d_head, hipStream_t stream) {
    const int st = check_split(dout, din, din, din, B, T, H, d_head);
    if (st != ATTN_SUCCESS) return st;
    HeadPtrs heads{{din, nullptr, nullptr}};
    clear_error();
    tcamd::launch_stripe_transpose(dout, ElemType::F32, nullptr, ElemType::F32, heads, true, B,
                                   T, 1, H, d_head, stream);
    return launch_status();
}

// ---- materialised softmax ---------------------------------------------------------------

namespace {

int softmax_fwd(const float* scores, float* probs, int B, int H, int T, float scale,
                int zero_block, hipStream_t stream) {
    if (scores == nullptr || probs == nullptr) return ATTN_ERROR_NULL_POINTER;
    if (B <= 0 || H <= 0 || T <= 0) return ATTN_ERROR_INVALID_DIM;
    if (!isfinite(scale) || zero_block < 0 || zero_block % 4 != 0)
        return ATTN_ERROR_INVALID_VALUE;
    const int64_t rows = static_cast<int64_t>(B) * H * T;
    if ((rows + 3) / 4 > kInt32Max) return ATTN_ERROR_INVALID_DIM;
    clear_error();
    tcamd::launch_causal_softmax_fwd_f32(scores, probs, rows, T, scale, stream, zero_block);
    return launch_status();
}

int softmax_bwd(const float* dprobs, const float* probs, float* dscores, int B, int H, int T,
                float scale, int zero_block, hipStream_t stream) {
    if (dprobs == nullptr || probs == nullptr || dscores == nullptr)
        return ATTN_ERROR_NULL_POINTER;
    if (B <= 0 || H <= 0 || T <= 0) return ATTN_ERROR_INVALID_DIM;
    if (!isfinite(scale) || zero_block < 0 || zero_block % 4 != 0)
        return ATTN_ERROR_INVALID_VALUE;
    const int64_t rows = static_cast<int64_t>(B) * H * T;
    if ((rows + 3) / 4 > kInt32Max) return ATTN_ERROR_INVALID_DIM;
    clear_error();
    tcamd::launch_causal_softmax_bwd_f32(dprobs, probs, dscores, rows, T, scale, stream,
                                         zero_block);
    return launch_status();
}

// The materialised attention's products read a probability (or dscores) row only up to the
// end of the 128-column block that holds its diagonal, so the softmax zeroes no further.
constexpr int kMatZeroBlock = 128;

}  // namespace

int attn_causal_softmax_forward_f32(const float* scores, float* probs, int B, int H, int T,
                                    float scale, hipStream_t stream) {
    return softmax_fwd(scores, probs, B, H, T, scale, 0, stream);
}

int attn_causal_softmax_backward_f32(const float* dprobs, const float* probs, float* dscores,
                                     int B, int H, int T, float scale, hipStream_t stream) {
    return softmax_bwd(dprobs, probs, dscores, B, H, T, scale, 0, stream);
}

int attn_causal_softmax_forward_blocked_f32(const float* scores, float* probs, int B, int H,
                                            int T, float scale, int zero_block,
                                            hipStream_t stream) {
    return softmax_fwd(scores, probs, B, H, T, scale, zero_block, stream);
}

int attn_causal_softmax_backward_blocked_f32(const float* dprobs, const float* probs,
                                             float* dscores, int B, int H, int T, float scale,
                                             int zero_block, hipStream_t stream) {
    return softmax_bwd(dprobs, probs, dscores, B, H, T, scale, zero_block, stream);
}

// ---- materialised path ------------------------------------------------------------------

int attn_matmul_batched_strided_f32(const float* A, const float* B, float* C, int M, int N,
                                    int K, long long strideA, long long strideB,
                                    long long strideC, int batch_count, int transA, int transB,
                                    float alpha, float beta, hipStream_t stream) {
    if (A == nullptr || B == nullptr || C == nullptr) return ATTN_ERROR_NULL_POINTER;
    if (M <= 0 || N <= 0 || K <= 0) return ATTN_ERROR_INVALID_DIM;
    if (batch_count <= 0 || strideA < 0 || strideB < 0 || strideC < 0)
        return ATTN_ERROR_INVALID_VALUE;
    if (!isfinite(alpha) || !isfinite(beta)) return ATTN_ERROR_INVALID_VALUE;
    const int64_t tiles = ((static_cast<int64_t>(M) + 63) / 64) * ((static_cast<int64_t>(N) + 63) / 64);
    if (tiles * batch_count > kInt32Max) return ATTN_ERROR_INVALID_DIM;
    clear_error();
    tcamd::launch_batched_gemm_f32(A, B, C, M, N, K, strideA, strideB, strideC, batch_count,
                                   transA != 0, transB != 0, alpha, beta, stream);
    return launch_status();
}

int attn_matmul_batched_strided_causal_f32(const float* A, const float* B, float* C, int M,
                                           int N, int K, long long strideA, long long strideB,
                                           long long strideC, int batch_count, int transA,
                                           int transB, int causal, hipStream_t stream) {
    if (A == nullptr || B == nullptr || C == nullptr) return ATTN_ERROR_NULL_POINTER;
    if (causal < ATTN_GEMM_FULL || causal > ATTN_GEMM_UPPER_A) return ATTN_ERROR_INVALID_VALUE;
    if (causal == ATTN_GEMM_LOWER_OUT && M != N) return ATTN_ERROR_INVALID_DIM;
    if ((causal == ATTN_GEMM_LOWER_A || causal == ATTN_GEMM_UPPER_A) && M != K)
        return ATTN_ERROR_INVALID_DIM;
    if (M <= 0 || N <= 0 || K <= 0) return ATTN_ERROR_INVALID_DIM;
    if (batch_count <= 0 || strideA < 0 || strideB < 0 || strideC < 0)
        return ATTN_ERROR_INVALID_VALUE;
    const int64_t tiles = ((static_cast<int64_t>(M) + 63) / 64) * ((static_cast<int64_t>(N) + 63) / 64);
    if (tiles * batch_count > kInt32Max) return ATTN_ERROR_INVALID_DIM;
    clear_error();
    tcamd::launch_batched_gemm_f32(A, B, C, M, N, K, strideA, strideB, strideC, batch_count,
                                   transA != 0, transB != 0, 1.0f, 0.0f, stream,
                                   static_cast<tcamd::GemmTri>(causal));
    return launch_status();
}

struct attn_gemm_context {
    int device;
};

int attn_gemm_create(attn_gemm_handle* handle) {
    if (handle == nullptr) return ATTN_ERROR_NULL_POINTER;
    *handle = nullptr;
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) {
        (void)hipGetLastError();
        return ATTN_ERROR_LAUNCH;
    }
    *handle = new attn_gemm_context{dev};
    return ATTN_SUCCESS;
}

int attn_gemm_destroy(attn_gemm_handle handle) {
    delete handle;
    return ATTN_SUCCESS;
}

int attn_gemm_device(attn_gemm_handle handle) { return handle == nullptr ? -1 : handle->device; }

int attn_matmul_batched_strided_f32_h(attn_gemm_handle handle, const float* A, const float* B,
                                      float* C, int M, int N, int K, long long strideA,
                                      long long strideB, long long strideC, int batch_count,
                                      int transA, int transB, float alpha, float beta,
                                      hipStream_t stream) {
    if (handle == nullptr) return ATTN_ERROR_NULL_POINTER;
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess) {
        (void)hipGetLastError();
        return ATTN_ERROR_LAUNCH;
    }
    if (dev != handle->device) return ATTN_ERROR_INVALID_VALUE;
    return attn_matmul_batched_strided_f32(A, B, C, M, N, K, strideA, strideB, strideC,
                                           batch_count, transA, transB, alpha, beta, stream);
}

int attn_materialized_causal_forward_f32(const float* q, const float* k, const float* v,
                                         float* scores, float* probs, float* out, int B, int H,
                                         int T, int d_head, float scale, hipStream_t stream) {
    if (q == nullptr || k == nullptr || v == nullptr || scores == nullptr ||
        probs == nullptr || out == nullptr)
        return ATTN_ERROR_NULL_POINTER;
    const int st = check_materialized(B, H, T, d_head, scale);
    if (st != ATTN_SUCCESS) return st;
    const int BH = B * H;
    const long long sh = static_cast<long long>(T) * d_head, ss = static_cast<long long>(T) * T;
    clear_error();
    // src/model.cu:314-320: scores = Q K^T (alpha 1; the scale is applied in the softmax).
    // The causal softmax reads only j <= i: tiles wholly above the diagonal are not computed.
    tcamd::launch_batched_gemm_f32(q, k, scores, T, T, d_head, sh, sh, ss, BH, false, true,
                                   1.0f, 0.0f, stream, tcamd::kGemmLowerOut);
    tcamd::launch_causal_softmax_fwd_f32(scores, probs, static_cast<int64_t>(BH) * T, T, scale,
                                         stream, kMatZeroBlock);
    // src/model.cu:326-332: out = probs V (probs is zero above the diagonal, up to where the
    // product reads it)
    tcamd::launch_batched_gemm_f32(probs, v, out, T, d_head, T, ss, sh, sh, BH, false, false,
                                   1.0f, 0.0f, stream, tcamd::kGemmLowerA);
    return launch_status();
}

int attn_materialized_causal_backward_f32(const float* q, const float* k, const float* v,
                                          const float* probs, const float* dout, float* dprobs,
                                          float* dscores, float* dq, float* dk, float* dv,
                                          int B, int H, int T, int d_head, float scale,
                                          hipStream_t stream) {
    if (q == nullptr || k == nullptr || v == nullptr || probs == nullptr || dout == nullptr ||
        dprobs == nullptr || dscores == nullptr || dq == nullptr || dk == nullptr ||
        dv == nullptr)
        return ATTN_ERROR_NULL_POINTER;
    const int st = check_materialized(B, H, T, d_head, scale);
    if (st != ATTN_SUCCESS) return st;
    const int BH = B * H;
    const long long sh = static_cast<long long>(T) * d_head, ss = static_cast<long long>(T) * T;
    clear_error();
    // src/model.cu:618-623: dprobs = dO V^T (the softmax backward reads only j <= i)
    tcamd::launch_batched_gemm_f32(dout, v, dprobs, T, T, d_head, sh, sh, ss, BH, false, true,
                                   1.0f, 0.0f, stream, tcamd::kGemmLowerOut);
    // :626-631: dv = probs^T dO (probs^T is zero below the diagonal)
    tcamd::launch_batched_gemm_f32(probs, dout, dv, T, d_head, T, ss, sh, sh, BH, true, false,
                                   1.0f, 0.0f, stream, tcamd::kGemmUpperA);
    // :634: dscores = softmax backward (scale inside; zero above the diagonal, up to where
    // the two products read it)
    tcamd::launch_causal_softmax_bwd_f32(dprobs, probs, dscores, static_cast<int64_t>(BH) * T,
                                         T, scale, stream, kMatZeroBlock);
    // :637-642: dq = dscores K;  :644-649: dk = dscores^T Q
    tcamd::launch_batched_gemm_f32(dscores, k, dq, T, d_head, T, ss, sh, sh, BH, false, false,
                                   1.0f, 0.0f, stream, tcamd::kGemmLowerA);
    tcamd::launch_batched_gemm_f32(dscores, q, dk, T, d_head, T, ss, sh, sh, BH, true, false,
                                   1.0f, 0.0f, stream, tcamd::kGemmUpperA);
    return launch_status();
}

// ---- tiled fp32 ------------------------------------------------------------------------

int attn_tiled_causal_forward_f32(const float* q, const float* k, const float* v, float* out,
                                  int B, int H, int T, int d_head, float scale, float* m_out,
                                  float* l_out, hipStream_t stream) {
    if (q == nullptr || k == nullptr || v == nullptr || out == nullptr)
        return ATTN_ERROR_NULL_POINTER;
    const int st = check_tiled(B, H, T, d_head, scale);
    if (st != ATTN_SUCCESS) return st;
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out))
        return ATTN_ERROR_MISALIGNED;
    clear_error();
    const tcamd::HeadView hm = tcamd::head_major_view(H, T, d_head);
    tcamd::launch_flash_fwd_f32(q, k, v, out, m_out, l_out, B * H, T, d_head, scale, hm, hm,
                                stream);
    return launch_status();
}

int attn_precompute_dot_do_o_f32(const float* dO, const float* O, float* D, int B, int H,
                                 int T, int d_head, hipStream_t stream) {
    if (dO == nullptr || O == nullptr || D == nullptr) return ATTN_ERROR_NULL_POINTER;
    const int st = check_dims4(B, H, T, d_head);
    if (st != ATTN_SUCCESS) return st;
    clear_error();
    tcamd::launch_dot_do_o_f32(dO, O, D, static_cast<int64_t>(B) * H * T, d_head, stream);
    return launch_status();
}

int attn_tiled_causal_backward_dq_f32(const float* q, const float* k, const float* v,
                                      const float* o, const float* do_ptr, const float* m_ptr,
                                      const float* l_ptr, float* dq, float* d_workspace, int B,
                                      int H, int T, int d_head, float scale,
                                      hipStream_t stream) {
    if (q == nullptr || k == nullptr || v == nullptr || o == nullptr || do_ptr == nullptr ||
        m_ptr == nullptr || l_ptr == nullptr || dq == nullptr || d_workspace == nullptr)
        return ATTN_ERROR_NULL_POINTER;
    const int st = check_tiled(B, H, T, d_head, scale);
    if (st != ATTN_SUCCESS) return st;
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o) ||
        !aligned16(do_ptr) || !aligned16(dq))
        return ATTN_ERROR_MISALIGNED;
    clear_error();
    const tcamd::HeadView hm = tcamd::head_major_view(H, T, d_head);
    tcamd::launch_flash_bwd_dq_f32(q, k, v, o, do_ptr, m_ptr, l_ptr, dq, d_workspace, B * H, T,
                                   d_head, scale, hm, hm, hm, stream);
    return launch_status();
}

int attn_tiled_causal_backward_dkdv_f32(const float* q, const float* k, const float* v,
                                        const float* do_ptr, const float* m_ptr,
                                        const float* l_ptr, const float* d_workspace, float* dk,
                                        float* dv, int B, int H, int T, int d_head, float scale,
                                        hipStream_t stream) {
    if (q == nullptr || k == nullptr || v == nullptr || do_ptr == nullptr || m_ptr == nullptr ||
        l_ptr == nullptr || d_workspace == nullptr || dk == nullptr || dv == nullptr)
        return ATTN_ERROR_NULL_POINTER;
    const int st = check_tiled(B, H, T, d_head, scale);
    if (st != ATTN_SUCCESS) return st;
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(do_ptr) ||
        !aligned16(dk) || !aligned16(dv))
        return ATTN_ERROR_MISALIGNED;
    clear_error();
    const tcamd::HeadView hm = tcamd::head_major_view(H, T, d_head);
    tcamd::launch_flash_bwd_dkdv_f32(q, k, v, do_ptr, m_ptr, l_ptr, d_workspace, dk, dv, B * H,
                                     T, d_head, scale, hm, hm, hm, stream);
    return launch_status();
}

int attn_tiled_causal_backward_f32(const float* q, const float* k, const float* v,
                                   const float* o, const float* do_ptr, const float* m_ptr,
                                   const float* l_ptr, float* dq, float* dk, float* dv,
                                   float* d_workspace, int B, int H, int T, int d_head,
                                   float scale, hipStream_t stream) {
    // Validate the second stage's own arguments before the first stage is enqueued.
    if (dk == nullptr || dv == nullptr) return ATTN_ERROR_NULL_POINTER;
    if (check_tiled(B, H, T, d_head, scale) == ATTN_SUCCESS && (!aligned16(dk) || !aligned16(dv)))
        return ATTN_ERROR_MISALIGNED;
    int st = attn_tiled_causal_backward_dq_f32(q, k, v, o, do_ptr, m_ptr, l_ptr, dq,
                                               d_workspace, B, H, T, d_head, scale, stream);
    if (st != ATTN_SUCCESS) return st;
    return attn_tiled_causal_backward_dkdv_f32(q, k, v, do_ptr, m_ptr, l_ptr, d_workspace, dk,
                                               dv, B, H, T, d_head, scale, stream);
}

// ---- tiled fp32 backward without a caller workspace ------------------------------------

namespace {

// D of attn_tiled_causal_backward_f32_noalloc.  In host code this name is not a device
// address: kernels get the address that hipGetSymbolAddress returns for the current device.
static __device__ __align__(256) float scratch[ATTN_NOALLOC_SCRATCH_FLOATS];

// Device address of `scratch` on the current device, looked up once per device (on the
// first call there, with that device current).  Null if the lookup fails.
float* scratch_ptr() {
    constexpr int kMaxDev = 64;
    static std::atomic<float*> cache[kMaxDev] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) {
        (void)hipGetLastError();
        return nullptr;
    }
    float* p = cache[dev].load(std::memory_order_acquire);
    if (p == nullptr) {
        void* addr = nullptr;
        if (hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch)) != hipSuccess || addr == nullptr) {
            (void)hipGetLastError();
            return nullptr;
        }
        p = static_cast<float*>(addr);
        cache[dev].store(p, std::memory_order_release);
    }
    return p;
}

}  // namespace

int attn_tiled_causal_backward_f32_noalloc(const float* q, const float* k, const float* v,
                                           const float* o, const float* do_ptr,
                                           const float* m_ptr, const float* l_ptr, float* dq,
                                           float* dk, float* dv, int B, int H, int T,
                                           int d_head, float scale, hipStream_t stream) {
    if (q == nullptr || k == nullptr || v == nullptr || o == nullptr || do_ptr == nullptr ||
        m_ptr == nullptr || l_ptr == nullptr || dq == nullptr || dk == nullptr || dv == nullptr)
        return ATTN_ERROR_NULL_POINTER;
    const int st = check_tiled(B, H, T, d_head, scale);
    if (st != ATTN_SUCCESS) return st;
    if (static_cast<int64_t>(B) * H * T > ATTN_NOALLOC_SCRATCH_FLOATS)
        return ATTN_ERROR_SCRATCH_LIMIT;
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o) ||
        !aligned16(do_ptr) || !aligned16(dq) || !aligned16(dk) || !aligned16(dv))
        return ATTN_ERROR_MISALIGNED;
    float* ws = scratch_ptr();
    if (ws == nullptr) return ATTN_ERROR_LAUNCH;
    // D is written by the first stage for every row before the second stage reads it, so the
    // scratch needs no clearing.
    return attn_tiled_causal_backward_f32(q, k, v, o, do_ptr, m_ptr, l_ptr, dq, dk, dv, ws, B,
                                          H, T, d_head, scale, stream);
}

// ---- tiled bf16 ------------------------------------------------------------------------

int attn_tiled_causal_forward_bf16(const attn_bf16* q, const attn_bf16* k, const attn_bf16* v,
                                   attn_bf16* out, int B, int H, int T, int d_head, float scale,
                                   float* m_out, float* l_out, hipStream_t stream) {
    if (q == nullptr || k == nullptr || v == nullptr || out == nullptr)
        return ATTN_ERROR_NULL_POINTER;
    const int st = check_tiled(B, H, T, d_head, scale);
    if (st != ATTN_SUCCESS) return st;
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out))
        return ATTN_ERROR_MISALIGNED;
    clear_error();
    const tcamd::HeadView hm = tcamd::head_major_view(H, T, d_head);
    tcamd::launch_flash_fwd_bf16(q, k, v, out, m_out, l_out, B * H, T, d_head, scale, hm, hm,
                                 stream);
    return launch_status();
}

int attn_tiled_causal_backward_dq_bf16(const attn_bf16* q, const attn_bf16* k,
                                       const attn_bf16* v, const attn_bf16* o,
                                       const attn_bf16* do_ptr, const float* m_ptr,
                                       const float* l_ptr, attn_bf16* dq, float* d_workspace,
                                       int B, int H, int T, int d_head, float scale,
                                       hipStream_t stream) {
    if (q == nullptr || k == nullptr || v == nullptr || o == nullptr || do_ptr == nullptr ||
        m_ptr == nullptr || l_ptr == nullptr || dq == nullptr || d_workspace == nullptr)
        return ATTN_ERROR_NULL_POINTER;
    const int st = check_tiled(B, H, T, d_head, scale);
    if (st != ATTN_SUCCESS) return st;
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o) ||
        !aligned16(do_ptr) || !aligned16(dq))
        return ATTN_ERROR_MISALIGNED;
    clear_error();
    const tcamd::HeadView hm = tcamd::head_major_view(H, T, d_head);
    tcamd::launch_flash_bwd_dq_bf16(q, k, v, o, do_ptr, m_ptr, l_ptr, dq, d_workspace, B * H,
                                    T, d_head, scale, hm, hm, hm, stream);
    return launch_status();
}

int attn_tiled_causal_backward_dkdv_bf16(const attn_bf16* q, const attn_bf16* k,
                                         const attn_bf16* v, const attn_bf16* do_ptr,
                                         const float* m_ptr, const float* l_ptr,
                                         const float* d_workspace, attn_bf16* dk, attn_bf16* dv,
                                         int B, int H, int T, int d_head, float scale,
                                         hipStream_t stream) {
    if (q == nullptr || k == nullptr || v == nullptr || do_ptr == nullptr || m_ptr == nullptr ||
        l_ptr == nullptr || d_workspace == nullptr || dk == nullptr || dv == nullptr)
        return ATTN_ERROR_NULL_POINTER;
    const int st = check_tiled(B, H, T, d_head, scale);
    if (st != ATTN_SUCCESS) return st;
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(do_ptr) ||
        !aligned16(dk) || !aligned16(dv))
        return ATTN_ERROR_MISALIGNED;
    clear_error();
    const tcamd::HeadView hm = tcamd::head_major_view(H, T, d_head);
    tcamd::launch_flash_bwd_dkdv_bf16(q, k, v, do_ptr, m_ptr, l_ptr, d_workspace, dk, dv,
                                      B * H, T, d_head, scale, hm, hm, hm, stream);
    return launch_status();
}

int attn_tiled_causal_backward_bf16(const attn_bf16* q, const attn_bf16* k,
                                    const attn_bf16* v, const attn_bf16* o,
                                    const attn_bf16* do_ptr, const float* m_ptr,
                                    const float* l_ptr, attn_bf16* dq, attn_bf16* dk,
                                    attn_bf16* dv, float* d_workspace, int B, int H, int T,
                                    int d_head, float scale, hipStream_t stream) {
    if (dk == nullptr || dv == nullptr) return ATTN_ERROR_NULL_POINTER;
    if (check_tiled(B, H, T, d_head, scale) == ATTN_SUCCESS && (!aligned16(dk) || !aligned16(dv)))
        return ATTN_ERROR_MISALIGNED;
    int st = attn_tiled_causal_backward_dq_bf16(q, k, v, o, do_ptr, m_ptr, l_ptr, dq,
                                                d_workspace, B, H, T, d_head, scale, stream);
    if (st != ATTN_SUCCESS) return st;
    return attn_tiled_causal_backward_dkdv_bf16(q, k, v, do_ptr, m_ptr, l_ptr, d_workspace, dk,
                                                dv, B, H, T, d_head, scale, stream);
}

// ---- packed QKV layout (split-transpose fused into the attention kernels) --------------

int attn_packed_causal_forward_f32(const float* qkv, float* out, int B, int H, int T,
                                   int d_head, float scale, float* m_out, float* l_out,
                                   hipStream_t stream) {
    return packed_forward(qkv, out, B, H, T, d_head, scale, m_out, l_out, false, stream);
}
int attn_packed_causal_backward_dq_f32(const float* qkv, const float* o, const float* do_ptr,
                                       const float* m_ptr, const float* l_ptr, float* dqkv,
                                       float* d_workspace, int B, int H, int T, int d_head,
                                       float scale, hipStream_t stream) {
    return packed_backward_dq(qkv, o, do_ptr, m_ptr, l_ptr, dqkv, d_workspace, B, H, T, d_head,
                              scale, false, stream);
}
int attn_packed_causal_backward_dkdv_f32(const float* qkv, const float* do_ptr,
                                         const float* m_ptr, const float* l_ptr,
                                         const float* d_workspace, float* dqkv, int B, int H,
                                         int T, int d_head, float scale, hipStream_t stream) {
    return packed_backward_dkdv(qkv, do_ptr, m_ptr, l_ptr, d_workspace, dqkv, B, H, T, d_head,
                                scale, false, stream);
}
int attn_packed_causal_backward_f32(const float* qkv, const float* o, const float* do_ptr,
                                    const float* m_ptr, const float* l_ptr, float* dqkv,
                                    float* d_workspace, int B, int H, int T, int d_head,
                                    float scale, hipStream_t stream) {
    return packed_backward(qkv, o, do_ptr, m_ptr, l_ptr, dqkv, d_workspace, B, H, T, d_head,
                           scale, false, stream);
}
int attn_packed_causal_forward_bf16(const attn_bf16* qkv, attn_bf16* out, int B, int H, int T,
                                    int d_head, float scale, float* m_out, float* l_out,
                                    hipStream_t stream) {
    return packed_forward(qkv, out, B, H, T, d_head, scale, m_out, l_out, false, stream);
}
int attn_packed_causal_backward_dq_bf16(const attn_bf16* qkv, const attn_bf16* o,
                                        const attn_bf16* do_ptr, const float* m_ptr,
                                        const float* l_ptr, attn_bf16* dqkv, float* d_workspace,
                                        int B, int H, int T, int d_head, float scale,
                                        hipStream_t stream) {
    return packed_backward_dq(qkv, o, do_ptr, m_ptr, l_ptr, dqkv, d_workspace, B, H, T, d_head,
                              scale, false, stream);
}
int attn_packed_causal_backward_dkdv_bf16(const attn_bf16* qkv, const attn_bf16* do_ptr,
                                          const float* m_ptr, const float* l_ptr,
                                          const float* d_workspace, attn_bf16* dqkv, int B,
                                          int H, int T, int d_head, float scale,
                                          hipStream_t stream) {
    return packed_backward_dkdv(qkv, do_ptr, m_ptr, l_ptr, d_workspace, dqkv, B, H, T, d_head,
                                scale, false, stream);
}
int attn_packed_causal_backward_bf16(const attn_bf16* qkv, const attn_bf16* o,
                                     const attn_bf16* do_ptr, const float* m_ptr,
                                     const float* l_ptr, attn_bf16* dqkv, float* d_workspace,
                                     int B, int H, int T, int d_head, float scale,
                                     hipStream_t stream) {
    return packed_backward(qkv, o, do_ptr, m_ptr, l_ptr, dqkv, d_workspace, B, H, T, d_head,
                           scale, false, stream);
}

// ---- fused: packed QKV in, heads merged out (split-transpose and head merge fused) -------

int attn_fused_causal_forward_f32(const float* qkv, float* out, int B, int H, int T,
                                  int d_head, float scale, float* m_out, float* l_out,
                                  hipStream_t stream) {
    return packed_forward(qkv, out, B, H, T, d_head, scale, m_out, l_out, true, stream);
}
int attn_fused_causal_backward_dq_f32(const float* qkv, const float* o, const float* do_ptr,
                                      const float* m_ptr, const float* l_ptr, float* dqkv,
                                      float* d_workspace, int B, int H, int T, int d_head,
                                      float scale, hipStream_t stream) {
    return packed_backward_dq(qkv, o, do_ptr, m_ptr, l_ptr, dqkv, d_workspace, B, H, T, d_head,
                              scale, true, stream);
}
int attn_fused_causal_backward_dkdv_f32(const float* qkv, const float* do_ptr,
                                        const float* m_ptr, const float* l_ptr,
                                        const float* d_workspace, float* dqkv, int B, int H,
                                        int T, int d_head, float scale, hipStream_t stream) {
    return packed_backward_dkdv(qkv, do_ptr, m_ptr, l_ptr, d_workspace, dqkv, B, H, T, d_head,
                                scale, true, stream);
}
int attn_fused_causal_backward_f32(const float* qkv, const float* o, const float* do_ptr,
                                   const float* m_ptr, const float* l_ptr, float* dqkv,
                                   float* d_workspace, int B, int H, int T, int d_head,
                                   float scale, hipStream_t stream) {
    return packed_backward(qkv, o, do_ptr, m_ptr, l_ptr, dqkv, d_workspace, B, H, T, d_head,
                           scale, true, stream);
}
int attn_fused_causal_forward_bf16(const attn_bf16* qkv, attn_bf16* out, int B, int H, int T,
                                   int d_head, float scale, float* m_out, float* l_out,
                                   hipStream_t stream) {
    return packed_forward(qkv, out, B, H, T, d_head, scale, m_out, l_out, true, stream);
}
int attn_fused_causal_backward_dq_bf16(const attn_bf16* qkv, const attn_bf16* o,
                                       const attn_bf16* do_ptr, const float* m_ptr,
                                       const float* l_ptr, attn_bf16* dqkv, float* d_workspace,
                                       int B, int H, int T, int d_head, float scale,
                                       hipStream_t stream) {
    return packed_backward_dq(qkv, o, do_ptr, m_ptr, l_ptr, dqkv, d_workspace, B, H, T, d_head,
                              scale, true, stream);
}
int attn_fused_causal_backward_dkdv_bf16(const attn_bf16* qkv, const attn_bf16* do_ptr,
                                         const float* m_ptr, const float* l_ptr,
                                         const float* d_workspace, attn_bf16* dqkv, int B,
                                         int H, int T, int d_head, float scale,
                                         hipStream_t stream) {
    return packed_backward_dkdv(qkv, do_ptr, m_ptr, l_ptr, d_workspace, dqkv, B, H, T, d_head,
                                scale, true, stream);
}
int attn_fused_causal_backward_bf16(const attn_bf16* qkv, const attn_bf16* o,
                                    const attn_bf16* do_ptr, const float* m_ptr,
                                    const float* l_ptr, attn_bf16* dqkv, float* d_workspace,
                                    int B, int H, int T, int d_head, float scale,
                                    hipStream_t stream) {
    return packed_backward(qkv, o, do_ptr, m_ptr, l_ptr, dqkv, d_workspace, B, H, T, d_head,
                           scale, true, stream);
}


// ---- fp32 on bf16 MFMAs (three bf16 planes per operand) --------------------------------

size_t attn_f32_ds_workspace_bytes(int B, int H, int T, int d_head) {
    if (B <= 0 || H <= 0 || T <= 0 || d_head <= 0) return 0;
    return ds_f32_elems(B, H, T) * sizeof(float);
}

int attn_f32_backward_uses_ds(int B, int H, int T, int d_head) {
    if (d_head != 32 && d_head != 64 && d_head != 128) return 0;
    const size_t bytes = attn_f32_ds_workspace_bytes(B, H, T, d_head);
    return bytes != 0 && bytes <= kDsMaxBytes ? 1 : 0;
}

int attn_packed_causal_backward_ds_f32(const float* qkv, const float* o, const float* do_ptr,
                                       const float* m_ptr, const float* l_ptr, float* dqkv,
                                       float* d_workspace, float* ds_workspace, int B, int H,
                                       int T, int d_head, float scale, hipStream_t stream) {
    return packed_backward_ds_f32(qkv, o, do_ptr, m_ptr, l_ptr, dqkv, d_workspace, ds_workspace,
                                  B, H, T, d_head, scale, false, stream);
}
int attn_fused_causal_backward_ds_f32(const float* qkv, const float* o, const float* do_ptr,
                                      const float* m_ptr, const float* l_ptr, float* dqkv,
                                      float* d_workspace, float* ds_workspace, int B, int H,
                                      int T, int d_head, float scale, hipStream_t stream) {
    return packed_backward_ds_f32(qkv, o, do_ptr, m_ptr, l_ptr, dqkv, d_workspace, ds_workspace,
                                  B, H, T, d_head, scale, true, stream);
}
int attn_packed_causal_backward_prep_f32(const float* o, const float* do_ptr, float* d_workspace,
                                         int B, int H, int T, int d_head, hipStream_t stream) {
    return packed_backward_prep_f32(o, do_ptr, d_workspace, B, H, T, d_head, false, stream);
}
int attn_fused_causal_backward_prep_f32(const float* o, const float* do_ptr, float* d_workspace,
                                        int B, int H, int T, int d_head, hipStream_t stream) {
    return packed_backward_prep_f32(o, do_ptr, d_workspace, B, H, T, d_head, true, stream);
}
int attn_packed_causal_backward_dkdv_ds_f32(const float* qkv, const float* do_ptr,
                                            const float* m_ptr, const float* l_ptr,
                                            const float* d_workspace, float* dqkv,
                                            float* ds_workspace, int B, int H, int T,
                                            int d_head, float scale, hipStream_t stream) {
    return packed_backward_dkdv_ds_f32(qkv, do_ptr, m_ptr, l_ptr, d_workspace, dqkv,
                                       ds_workspace, B, H, T, d_head, scale, false, stream);
}
int attn_fused_causal_backward_dkdv_ds_f32(const float* qkv, const float* do_ptr,
                                           const float* m_ptr, const float* l_ptr,
                                           const float* d_workspace, float* dqkv,
                                           float* ds_workspace, int B, int H, int T, int d_head,
                                           float scale, hipStream_t stream) {
    return packed_backward_dkdv_ds_f32(qkv, do_ptr, m_ptr, l_ptr, d_workspace, dqkv,
                                       ds_workspace, B, H, T, d_head, scale, true, stream);
}
int attn_causal_backward_dq_ds_f32(const float* qkv, float* dqkv, const float* ds_workspace,
                                   int B, int H, int T, int d_head, float scale,
                                   hipStream_t stream) {
    return backward_dq_ds_f32(qkv, dqkv, ds_workspace, B, H, T, d_head, scale, stream);
}

size_t attn_f32x3_planes_bytes(int B, int H, int T, int d_head) {
    if (B <= 0 || H <= 0 || T <= 0 || d_head <= 0) return 0;
    return static_cast<size_t>(kPlaneTensors) * kPlanes * plane_elems(B, H, T, d_head) *
           sizeof(uint16_t);
}

size_t attn_f32x3_ds_workspace_bytes(int B, int H, int T, int d_head) {
    if (B <= 0 || H <= 0 || T <= 0 || d_head <= 0 || !uses_ds(B, H, T, d_head)) return 0;
    return ds_elems(B, H, T) * sizeof(float);
}

size_t attn_f32x3_workspace_bytes(int B, int H, int T, int d_head) {
    return attn_f32x3_planes_bytes(B, H, T, d_head) +
           attn_f32x3_ds_workspace_bytes(B, H, T, d_head);
}

int attn_f32x3_backward_uses_ds(int B, int H, int T, int d_head) {
    if (B <= 0 || H <= 0 || T <= 0 || d_head <= 0) return 0;
    return uses_ds(B, H, T, d_head) ? 1 : 0;
}

int attn_packed_causal_forward_f32x3(const float* qkv, float* out, int B, int H, int T,
                                     int d_head, float scale, float* m_out, float* l_out,
                                     void* planes, hipStream_t stream) {
    return packed_forward_f32x3(qkv, out, B, H, T, d_head, scale, m_out, l_out, planes, false,
                                stream);
}

int attn_fused_causal_forward_f32x3(const float* qkv, float* out, int B, int H, int T,
                                    int d_head, float scale, float* m_out, float* l_out,
                                    void* planes, hipStream_t stream) {
    return packed_forward_f32x3(qkv, out, B, H, T, d_head, scale, m_out, l_out, planes, true,
                                stream);
}

int attn_packed_causal_backward_f32x3(const float* qkv, const float* o, const float* do_ptr,
                                      const float* m_ptr, const float* l_ptr, float* dqkv,
                                      float* d_workspace, int B, int H, int T, int d_head,
                                      float scale, void* planes, int kv_planes_ready,
                                      hipStream_t stream) {
    return packed_backward_f32x3(qkv, o, do_ptr, m_ptr, l_ptr, dqkv, d_workspace, B, H, T,
                                 d_head, scale, planes, combined_ds(planes, B, H, T, d_head),
                                 kv_planes_ready, false, stream);
}

int attn_fused_causal_backward_f32x3(const float* qkv, const float* o, const float* do_ptr,
                                     const float* m_ptr, const float* l_ptr, float* dqkv,
                                     float* d_workspace, int B, int H, int T, int d_head,
                                     float scale, void* planes, int kv_planes_ready,
                                     hipStream_t stream) {
    return packed_backward_f32x3(qkv, o, do_ptr, m_ptr, l_ptr, dqkv, d_workspace, B, H, T,
                                 d_head, scale, planes, combined_ds(planes, B, H, T, d_head),
                                 kv_planes_ready, true, stream);
}

int attn_packed_causal_backward_ds_f32x3(const float* qkv, const float* o, const float* do_ptr,
                                         const float* m_ptr, const float* l_ptr, float* dqkv,
                                         float* d_workspace, float* ds_workspace, int B, int H,
                                         int T, int d_head, float scale, void* planes,
                                         int kv_planes_ready, hipStream_t stream) {
    return packed_backward_f32x3(qkv, o, do_ptr, m_ptr, l_ptr, dqkv, d_workspace, B, H, T,
                                 d_head, scale, planes, ds_workspace, kv_planes_ready, false,
                                 stream);
}

int attn_fused_causal_backward_ds_f32x3(const float* qkv, const float* o, const float* do_ptr,
                                        const float* m_ptr, const float* l_ptr, float* dqkv,
                                        float* d_workspace, float* ds_workspace, int B, int H,
                                        int T, int d_head, float scale, void* planes,
                                        int kv_planes_ready, hipStream_t stream) {
    return packed_backward_f32x3(qkv, o, do_ptr, m_ptr, l_ptr, dqkv, d_workspace, B, H, T,
                                 d_head, scale, planes, ds_workspace, kv_planes_ready, true,
                                 stream);
}

int attn_packed_causal_backward_prep_f32x3(const float* qkv, const float* o,
                                           const float* do_ptr, float* d_workspace, int B,
                                           int H, int T, int d_head, void* planes,
                                           int kv_planes_ready, hipStream_t stream) {
    return packed_backward_prep_f32x3(qkv, o, do_ptr, d_workspace, B, H, T, d_head, planes,
                                      kv_planes_ready, false, stream);
}

int attn_fused_causal_backward_prep_f32x3(const float* qkv, const float* o, const float* do_ptr,
                                          float* d_workspace, int B, int H, int T, int d_head,
                                          void* planes, int kv_planes_ready,
                                          hipStream_t stream) {
    return packed_backward_prep_f32x3(qkv, o, do_ptr, d_workspace, B, H, T, d_head, planes,
                                      kv_planes_ready, true, stream);
}

int attn_causal_backward_dkdv_ds_f32x3(const float* qkv, const float* m_ptr, const float* l_ptr,
                                       const float* d_workspace, float* dqkv, int B, int H,
                                       int T, int d_head, float scale, void* planes,
                                       hipStream_t stream) {
    return packed_backward_dkdv_ds_f32x3(qkv, m_ptr, l_ptr, d_workspace, dqkv, B, H, T, d_head,
                                         scale, planes, combined_ds(planes, B, H, T, d_head),
                                         stream);
}

int attn_causal_backward_dq_ds_f32x3(float* dqkv, int B, int H, int T, int d_head, float scale,
                                     const void* planes, hipStream_t stream) {
    return packed_backward_dq_ds_f32x3(
        dqkv, B, H, T, d_head, scale, planes,
        combined_ds(const_cast<void*>(planes), B, H, T, d_head), stream);
}

int attn_packed_causal_backward_dq_f32x3(const float* qkv, const float* o,
                                         const float* do_ptr, const float* m_ptr,
                                         const float* l_ptr, float* dqkv, float* d_workspace,
                                         int B, int H, int T, int d_head, float scale,
                                         void* planes, int kv_planes_ready,
                                         hipStream_t stream) {
    return packed_backward_dq_f32x3(qkv, o, do_ptr, m_ptr, l_ptr, dqkv, d_workspace, B, H, T,
                                    d_head, scale, planes, kv_planes_ready, false, stream);
}

int attn_fused_causal_backward_dq_f32x3(const float* qkv, const float* o, const float* do_ptr,
                                        const float* m_ptr, const float* l_ptr, float* dqkv,
                                        float* d_workspace, int B, int H, int T, int d_head,
                                        float scale, void* planes, int kv_planes_ready,
                                        hipStream_t stream) {
    return packed_backward_dq_f32x3(qkv, o, do_ptr, m_ptr, l_ptr, dqkv, d_workspace, B, H, T,
                                    d_head, scale, planes, kv_planes_ready, true, stream);
}

int attn_causal_backward_dkdv_f32x3(const float* qkv, const float* m_ptr, const float* l_ptr,
                                    const float* d_workspace, float* dqkv, int B, int H, int T,
                                    int d_head, float scale, const void* planes,
                                    hipStream_t stream) {
    return packed_backward_dkdv_f32x3(qkv, m_ptr, l_ptr, d_workspace, dqkv, B, H, T, d_head,
                                      scale, planes, stream);
}

int attn_tiled_causal_forward_f32x3(const float* q, const float* k, const float* v,
                                    float* out, int B, int H, int T, int d_head, float scale,
                                    float* m_out, float* l_out, void* planes,
                                    hipStream_t stream) {
    return tiled_forward_f32x3(q, k, v, out, B, H, T, d_head, scale, m_out, l_out, planes,
                               stream);
}

int attn_tiled_causal_backward_dq_f32x3(const float* q, const float* k, const float* v,
                                        const float* o, const float* do_ptr,
                                        const float* m_ptr, const float* l_ptr, float* dq,
                                        float* d_workspace, int B, int H, int T, int d_head,
                                        float scale, void* planes, int kv_planes_ready,
                                        hipStream_t stream) {
    return tiled_backward_dq_f32x3(q, k, v, o, do_ptr, m_ptr, l_ptr, dq, d_workspace, B, H, T,
                                   d_head, scale, planes, kv_planes_ready, stream);
}

int attn_tiled_causal_backward_dkdv_f32x3(const float* k, const float* v, const float* m_ptr,
                                          const float* l_ptr, const float* d_workspace,
                                          float* dk, float* dv, int B, int H, int T,
                                          int d_head, float scale, const void* planes,
                                          hipStream_t stream) {
    return tiled_backward_dkdv_f32x3(k, v, m_ptr, l_ptr, d_workspace, dk, dv, B, H, T, d_head,
                                     scale, planes, stream);
}

int attn_tiled_causal_backward_f32x3(const float* q, const float* k, const float* v,
                                     const float* o, const float* do_ptr, const float* m_ptr,
                                     const float* l_ptr, float* dq, float* dk, float* dv,
                                     float* d_workspace, int B, int H, int T, int d_head,
                                     float scale, void* planes, int kv_planes_ready,
                                     hipStream_t stream) {
    return tiled_backward_f32x3(q, k, v, o, do_ptr, m_ptr, l_ptr, dq, dk, dv, d_workspace, B, H,
                                T, d_head, scale, planes, kv_planes_ready, stream);
}

}  // extern "C"
