// device_common.hpp - gfx950 (CDNA4) device helpers shared by the attention kernels.
//
// Wavefronts are 64 lanes.  The 32x32 MFMA ops used here see a wave as two halves of 32
// lanes: lane l supplies row/column (l & 31) of an operand and k-slot group (l >> 5).
// Their 32x32 fp32 result lands in 16 registers per lane:
//     acc[v] of lane l  =  D[row = 8*(v/4) + 4*(l/32) + (v%4)][col = l%32]
// (the layout AMD documents for v_mfma_f32_32x32x{2f32,16_bf16}).  acc_row() below is
// that map; every kernel derives its masks and LDS addresses from it.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tcamd {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;

// Row of D held by register v of a lane in half `half` (= lane >> 5), 32x32 MFMA layout.
__device__ __forceinline__ constexpr int acc_row(int v, int half) {
    return 8 * (v >> 2) + 4 * half + (v & 3);
}

// D(32x32) += A(32x2) * B(2x32).  a = A[l%32][l/32], b = B[l/32][l%32].
__device__ __forceinline__ f32x16 mfma_32x32x2_f32(float a, float b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// D(32x32) += A(32x16) * B(16x32), bf16 operands, fp32 accumulate.  Lane l supplies eight
// k-values of row l%32 of A and column l%32 of B from k-group l/32; A and B only have to
// agree on which k each (group, element) slot carries.
__device__ __forceinline__ f32x16 mfma_32x32x16_bf16(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Combine the two 32-lane halves of a wave with v_permlane32_swap: after the swap the
// two results hold x[l%32] and x[l%32 + 32] in some order, so max/sum of them is the same
// value in lanes l and l^32.
__device__ __forceinline__ float xhalf_max(float x) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                              false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xhalf_sum(float x) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                              false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Where head bh = b*H + h of a (B, H, T, d) operand lives: element (t, e) is at
// off(bh) + t*row + e.  Head-major tensors (B, H, T, d): batch = H*T*d, head = T*d, row = d.
// The packed QKV layout (B, T, 3*H*d), pointer advanced to the q, k or v column block:
// batch = 3*H*T*d, head = d, row = 3*H*d.  The merged-heads layout (B, T, H*d) of the
// attention output: batch = H*T*d, head = d, row = H*d.
struct HeadView {
    long long batch;
    long long head;
    int row;
    int H;
    __device__ __forceinline__ size_t off(int bh) const {
        return static_cast<size_t>((bh / H) * batch + (bh % H) * head);
    }
};
inline HeadView head_major_view(int H, int T, int d) {
    return HeadView{static_cast<long long>(H) * T * d, static_cast<long long>(T) * d, d, H};
}
inline HeadView packed_qkv_view(int H, int T, int d) {
    return HeadView{3LL * H * T * d, d, 3 * H * d, H};
}
inline HeadView merged_view(int H, int T, int d) {
    return HeadView{static_cast<long long>(H) * T * d, d, H * d, H};
}

// fp32 -> bf16 bits, round to nearest even (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float x) {
    __bf16 h = static_cast<__bf16>(x);
    return __builtin_bit_cast(uint16_t, h);
}
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
    return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Map a linear workgroup id so that consecutive logical ids stay on one XCD.  The
// dispatcher hands workgroup i to XCD i % 8; with n % 8 == 0 this returns a permutation
// whose block of n/8 consecutive logical ids all run on the same XCD (same L2).
__device__ __forceinline__ int xcd_swizzle(int id, int n) {
    if ((n & 7) != 0) return id;
    return (id & 7) * (n >> 3) + (id >> 3);
}

}  // namespace tcamd
