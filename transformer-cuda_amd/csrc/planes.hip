// planes.hip - fp32 tensors into three bf16 planes (HBM-bound), the operand format of the
// fp32 attention kernels that run on bf16 MFMAs (flash_bf16*.hip with NP = 3).
//
// Element x of a (B*H, T, d) fp32 view becomes x_0 = bf16(x), x_1 = bf16(x - x_0),
// x_2 = bf16(x - x_0 - x_1) (round to nearest even), written to three head-major bf16
// tensors pstride elements apart.  A thread moves 8 consecutive elements of a row: two
// 16-byte loads, three 16-byte nontemporal stores (the planes are next read by other
// kernels, not from this kernel's L2 lines).
#include "bf16_tile.hpp"
#include "device_common.hpp"
#include "launch.hpp"

namespace tcamd {
namespace {

constexpr int kThreads = 256;

// ntens tensors in one launch: tensor j reads src + j*src_step and writes dst + j*dst_step.
__global__ __launch_bounds__(kThreads) void split_planes_kernel(
    const float* __restrict__ src, HeadView sv, uint16_t* __restrict__ dst, size_t pstride,
    int T, int d, long long units, int ntens, size_t src_step, size_t dst_step) {
    const int upr = d / 8;  // 8-element units per row
    for (long long w = blockIdx.x * static_cast<long long>(kThreads) + threadIdx.x;
         w < units * ntens; w += static_cast<long long>(gridDim.x) * kThreads) {
        const int j = static_cast<int>(w / units);
        const long long u = w - j * units;
        const float* src_j = src + j * src_step;
        uint16_t* dst_j = dst + j * dst_step;
        const long long row = u / upr;
        const int c = static_cast<int>(u - row * upr) * 8;
        const int bh = static_cast<int>(row / T);
        const int t = static_cast<int>(row - static_cast<long long>(bh) * T);
        const float* p = src_j + sv.off(bh) + static_cast<size_t>(t) * sv.row + c;
        const f32x4 a = *reinterpret_cast<const f32x4*>(p);
        const f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
        const float x[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
        bf16x8 pl[3];
        bf16t::split_planes<3>(x, pl);
        uint16_t* o = dst_j + static_cast<size_t>(row) * d + c;  // head-major
#pragma unroll
        for (int i = 0; i < 3; ++i)
            __builtin_nontemporal_store(__builtin_bit_cast(u16x8, pl[i]),
                                        reinterpret_cast<u16x8*>(o + i * pstride));
    }
}

}  // namespace

void launch_split_planes(const float* src, const HeadView& sv, uint16_t* dst, size_t pstride,
                         int BH, int T, int d, hipStream_t stream, int ntens, size_t src_step,
                         size_t dst_step) {
    const long long units = static_cast<long long>(BH) * T * (d / 8);
    if (units == 0 || ntens <= 0) return;
    const long long want = (units * ntens + kThreads - 1) / kThreads;
    const int grid = static_cast<int>(want < 16384 ? want : 16384);
    hipLaunchKernelGGL(split_planes_kernel, dim3(grid), dim3(kThreads), 0, stream, src, sv, dst,
                       pstride, T, d, units, ntens, src_step, dst_step);
}

}  // namespace tcamd
