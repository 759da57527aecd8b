// batched_gemm.hip - strided-batched fp32 GEMM on v_mfma_f32_32x32x2_f32, the contraction of
// the reference's materialised attention mode.
//
// Reference: matmul_batched_strided (src/kernels/matmul.cu:167-207, declared
// include/kernels/matmul.cuh:44), which calls cublasSgemmStridedBatched.  Same semantics,
// row-major: for every batch b,
//     C_b (M x N, ldc = N) = alpha * op(A_b) * op(B_b) + beta * C_b
// with op(A) = A (M x K, lda = K) or A^T (A stored K x M, lda = M), op(B) = B (K x N,
// ldb = N) or B^T (B stored N x K, ldb = K).  beta == 0 does not read C (BLAS convention).
//
// A workgroup of 4 waves computes a 64 x 64 tile of C; wave (wm, wn) owns the 32 x 32
// quarter (wm, wn) in one MFMA accumulator.  K advances in 16-deep chunks staged through
// LDS (double buffered, the next chunk's global loads in flight during the current chunk's
// 8 MFMAs per wave).  LDS holds both operands k-major (As[k][m], Bs[k][n]), so an MFMA
// operand read is 32 consecutive floats per k.  Loads are scalar with bounds checks, which
// serves every (trans, size, alignment) combination the reference's call sites produce.
#include <stdint.h>

#include "device_common.hpp"
#include "launch.hpp"

namespace tcamd {
namespace {

constexpr int kBM = 64, kBN = 64, kBK = 16, kPad = 4;
constexpr int kThreads = 256;
constexpr int kLoads = kBM * kBK / kThreads;  // elements of each operand per thread per chunk

template <bool TA, bool TB>
__global__ __launch_bounds__(kThreads) void bgemm_f32_kernel(
    const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, int M,
    int N, int K, long long sA, long long sB, long long sC, float alpha, float beta,
    int tiles_m, int tiles_n) {
    __shared__ float As[2][kBK][kBM + kPad];
    __shared__ float Bs[2][kBK][kBN + kPad];
    const long long tiles = static_cast<long long>(tiles_m) * tiles_n;
    const long long id = blockIdx.x;
    const long long batch = id / tiles;
    const int t = static_cast<int>(id - batch * tiles);
    const int m0 = (t / tiles_n) * kBM;
    const int n0 = (t % tiles_n) * kBN;
    const float* Ab = A + batch * sA;
    const float* Bb = B + batch * sB;
    float* Cb = C + batch * sC;
    const int lda = TA ? M : K;
    const int ldb = TB ? K : N;

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    // Element i of this thread in a chunk: (kk, mm) of A and (kk, nn) of B, chosen so that
    // consecutive threads read consecutive addresses of the stored layout.
    int a_k[kLoads], a_m[kLoads], b_k[kLoads], b_n[kLoads];
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
        const int e = tid + kThreads * i;
        if (TA) { a_k[i] = e / kBM; a_m[i] = e % kBM; }   // stored K x M: m fastest
        else    { a_m[i] = e / kBK; a_k[i] = e % kBK; }   // stored M x K: k fastest
        if (TB) { b_n[i] = e / kBK; b_k[i] = e % kBK; }   // stored N x K: k fastest
        else    { b_k[i] = e / kBN; b_n[i] = e % kBN; }   // stored K x N: n fastest
    }
    float ra[kLoads], rb[kLoads];
    auto load = [&](int k0) {
#pragma unroll
        for (int i = 0; i < kLoads; ++i) {
            const int m = m0 + a_m[i], k = k0 + a_k[i];
            ra[i] = (m < M && k < K)
                        ? Ab[TA ? static_cast<long long>(k) * lda + m
                                : static_cast<long long>(m) * lda + k]
                        : 0.0f;
            const int n = n0 + b_n[i], kb = k0 + b_k[i];
            rb[i] = (n < N && kb < K)
                        ? Bb[TB ? static_cast<long long>(n) * ldb + kb
                                : static_cast<long long>(kb) * ldb + n]
                        : 0.0f;
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int i = 0; i < kLoads; ++i) {
            As[buf][a_k[i]][a_m[i]] = ra[i];
            Bs[buf][b_k[i]][b_n[i]] = rb[i];
        }
    };

    f32x16 acc = f32x16{};
    const int nk = (K + kBK - 1) / kBK;
    load(0);
    store(0);
    __syncthreads();
    const int ar = 32 * wm + (lane & 31);
    const int bc = 32 * wn + (lane & 31);
    const int kh = lane >> 5;
    for (int kc = 0; kc < nk; ++kc) {
        const int buf = kc & 1;
        if (kc + 1 < nk) load((kc + 1) * kBK);
#pragma unroll
        for (int s = 0; s < kBK / 2; ++s)
            acc = mfma_32x32x2_f32(As[buf][2 * s + kh][ar], Bs[buf][2 * s + kh][bc], acc);
        if (kc + 1 < nk) store(buf ^ 1);
        __syncthreads();
    }

    const int col = n0 + bc;
    if (col < N) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int row = m0 + 32 * wm + acc_row(v, kh);
            if (row < M) {
                float* p = Cb + static_cast<long long>(row) * N + col;
                *p = beta == 0.0f ? alpha * acc[v] : fmaf(alpha, acc[v], beta * *p);
            }
        }
    }
}

}  // namespace

void launch_batched_gemm_f32(const float* A, const float* B, float* C, int M, int N, int K,
                             long long sA, long long sB, long long sC, int batch, bool transA,
                             bool transB, float alpha, float beta, hipStream_t stream) {
    const int tiles_m = (M + kBM - 1) / kBM;
    const int tiles_n = (N + kBN - 1) / kBN;
    const long long grid = static_cast<long long>(tiles_m) * tiles_n * batch;
    const dim3 g(static_cast<unsigned>(grid)), b(kThreads);
    if (transA) {
        if (transB)
            hipLaunchKernelGGL((bgemm_f32_kernel<true, true>), g, b, 0, stream, A, B, C, M, N,
                               K, sA, sB, sC, alpha, beta, tiles_m, tiles_n);
        else
            hipLaunchKernelGGL((bgemm_f32_kernel<true, false>), g, b, 0, stream, A, B, C, M, N,
                               K, sA, sB, sC, alpha, beta, tiles_m, tiles_n);
    } else {
        if (transB)
            hipLaunchKernelGGL((bgemm_f32_kernel<false, true>), g, b, 0, stream, A, B, C, M, N,
                               K, sA, sB, sC, alpha, beta, tiles_m, tiles_n);
        else
            hipLaunchKernelGGL((bgemm_f32_kernel<false, false>), g, b, 0, stream, A, B, C, M,
                               N, K, sA, sB, sC, alpha, beta, tiles_m, tiles_n);
    }
}

}  // namespace tcamd
