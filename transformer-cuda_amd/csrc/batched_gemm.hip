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
//
// When the operands allow 16-byte loads (the contiguous dimension of each operand a
// multiple of 4 elements, 16-byte aligned bases and batch strides: every call of the
// materialised attention with d_head % 4 == 0 and T % 4 == 0), a second kernel runs: each
// wave computes 64 x 64 of C as 2 x 2 MFMA blocks (every LDS operand read feeds two MFMAs)
// in a 128 x 128 workgroup tile, or 32 x 64 in a 128 x 64 tile for N <= 64, and global loads
// move 16 bytes per lane.  Where K is also a multiple of 16 (every materialised attention
// call with d_head % 16 == 0 and T % 16 == 0), the copy-pipelined kernel below replaces it:
// operand tiles go HBM -> LDS directly with up to three k chunks in flight, workgroups are
// laid out so that each XCD works through a contiguous range of tiles, and the causal forms
// enumerate only the tiles the mask leaves (square output) or pair long and short row tiles
// (triangular A, 64 x 64 tiles).
#include <stdint.h>

#include <type_traits>

#include "device_common.hpp"
#include "launch.hpp"
#include "lds_dma.hpp"
#include "sched.hpp"

namespace tcamd {
namespace {

constexpr int kBM = 64, kBN = 64, kBK = 16, kPad = 4;
constexpr int kThreads = 256;
constexpr int kLoads = kBM * kBK / kThreads;  // elements of each operand per thread per chunk

template <bool TA, bool TB>
__global__ __launch_bounds__(kThreads) void bgemm_f32_kernel(
    const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, int M,
    int N, int K, long long sA, long long sB, long long sC, float alpha, float beta,
    int tiles_m, int tiles_n, int tri) {
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
    // k chunks kc0 .. nk-1: where op(A) is triangular, the chunks of its nonzero part only
    int kc0 = 0, nk = (K + kBK - 1) / kBK;
    if (tri == kGemmLowerA) nk = min(nk, (m0 + kBM + kBK - 1) / kBK);
    if (tri == kGemmUpperA) kc0 = min(nk, m0 / kBK);
    if (kc0 < nk) {
        load(kc0 * kBK);
        store(kc0 & 1);
    }
    __syncthreads();
    const int ar = 32 * wm + (lane & 31);
    const int bc = 32 * wn + (lane & 31);
    const int kh = lane >> 5;
    for (int kc = kc0; kc < nk; ++kc) {
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

// ---------------------------------------------------------------------------------------
// Tiled kernel (16-byte loads).  LDS holds each operand as rows of 16 floats (one m of A, or
// one n of B, over a 16-deep k chunk) with k permuted, kp(k) = 8*(k % 2) + k / 2, so that the
// MFMA lane (r, kh), which takes k = 2s + kh at step s, finds its 8 values of the chunk at
// kp = 8kh .. 8kh + 7: two 16-byte reads.  The 16-byte chunk c of row r sits at chunk slot
// c ^ ((r / 4) % 4), so the 16 lanes of a read (rows r .. r+15, one chunk) hit distinct banks.
// ---------------------------------------------------------------------------------------
constexpr int kTK = 16;  // k per chunk
typedef float f32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ int kperm(int k) { return (k & 1) * 8 + (k >> 1); }
// Float index of (row r, permuted k kp) in an operand tile.
__device__ __forceinline__ int op_off(int r, int kp) {
    return r * kTK + ((((kp >> 2) ^ (r >> 2)) & 3) << 2) + (kp & 3);
}

// WM waves along M, 4 / WM along N; each wave computes I x J MFMA blocks of 32 x 32.
// tri (GemmTri): the causal structure the caller guarantees (k chunks of 16 and tiles of
// 128 rows align with it, so a tile's k range is cut at chunk boundaries).
template <bool TA, bool TB, int WM, int I, int J>
__global__ __launch_bounds__(kThreads) void bgemm_f32_tiled_kernel(
    const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, int M,
    int N, int K, long long sA, long long sB, long long sC, float alpha, float beta,
    int tiles_m, int tiles_n, int tri) {
    constexpr int WN = 4 / WM;
    constexpr int BM = 32 * I * WM, BN = 32 * J * WN;
    constexpr int kA4 = BM * kTK / 4 / kThreads;  // float4 of A per thread per chunk
    constexpr int kB4 = BN * kTK / 4 / kThreads;
    __shared__ __attribute__((aligned(16))) float As[2][BM * kTK];
    __shared__ __attribute__((aligned(16))) float Bs[2][BN * kTK];
    const long long tiles = static_cast<long long>(tiles_m) * tiles_n;
    const long long id = blockIdx.x;
    const long long batch = id / tiles;
    const int t = static_cast<int>(id - batch * tiles);
    // lower-triangular A: the last row blocks carry the longest k ranges, so they go first
    const int mt = tri == kGemmLowerA ? tiles_m - 1 - t / tiles_n : t / tiles_n;
    const int m0 = mt * BM;
    const int n0 = (t % tiles_n) * BN;
    if (tri == kGemmLowerOut && n0 > m0 + BM - 1) return;  // the whole tile is above the diagonal
    const float* Ab = A + batch * sA;
    const float* Bb = B + batch * sB;
    float* Cb = C + batch * sC;
    const int lda = TA ? M : K;
    const int ldb = TB ? K : N;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid >> 6;
    const int wm = wave % WM, wn = wave / WM;

    // One operand tile (R rows of the operand's M or N, kTK k) from a row-major source:
    // KCONT: the source's rows run over k (element (r, k) at r*ld + k), else over r
    // (element (r, k) at k*ld + r).  Fragment f of this thread covers 4 consecutive
    // elements of the contiguous dimension.
    f32x4 ra[kA4], rb[kB4];
    auto load_op = [&](auto kcont, const float* src, int ld, int r0, int rlim, int k0, auto& reg,
                       auto nfrag) {
        constexpr bool KC = decltype(kcont)::value;
        constexpr int NF = decltype(nfrag)::value;
#pragma unroll
        for (int i = 0; i < NF; ++i) {
            const int f = tid + kThreads * i;
            int r, k;
            if constexpr (KC) { r = f >> 2; k = (f & 3) * 4; }
            else { k = f % kTK; r = (f / kTK) * 4; }
            const bool ok = (r0 + r < rlim) && (k0 + k < K);
            reg[i] = ok ? *reinterpret_cast<const f32x4*>(
                              src + (KC ? static_cast<long long>(r0 + r) * ld + (k0 + k)
                                        : static_cast<long long>(k0 + k) * ld + (r0 + r)))
                        : f32x4{};
        }
    };
    auto store_op = [&](auto kcont, float* dst, const auto& reg, auto nfrag) {
        constexpr bool KC = decltype(kcont)::value;
        constexpr int NF = decltype(nfrag)::value;
#pragma unroll
        for (int i = 0; i < NF; ++i) {
            const int f = tid + kThreads * i;
            if constexpr (KC) {  // k = 4q .. 4q+3 of row r: kp 2q, 2q+1 and 8+2q, 9+2q
                const int r = f >> 2, q = f & 3;
                *reinterpret_cast<f32x2*>(dst + op_off(r, 2 * q)) = f32x2{reg[i][0], reg[i][2]};
                *reinterpret_cast<f32x2*>(dst + op_off(r, 8 + 2 * q)) = f32x2{reg[i][1], reg[i][3]};
            } else {  // rows r .. r+3 at one k; 16 lanes: 16 k of the same rows
                const int k = f % kTK, r = (f / kTK) * 4;
                const int kp = kperm(k);
#pragma unroll
                for (int j = 0; j < 4; ++j) dst[op_off(r + j, kp)] = reg[i][j];
            }
        }
    };
    using KA = std::integral_constant<bool, !TA>;  // A (M x K): rows over k unless transposed
    using KB = std::integral_constant<bool, TB>;   // B (K x N): rows over k when transposed
    using NA = std::integral_constant<int, kA4>;
    using NB = std::integral_constant<int, kB4>;
    auto load = [&](int k0) {
        load_op(KA{}, Ab, lda, m0, M, k0, ra, NA{});
        load_op(KB{}, Bb, ldb, n0, N, k0, rb, NB{});
    };
    auto store = [&](int buf) {
        store_op(KA{}, As[buf], ra, NA{});
        store_op(KB{}, Bs[buf], rb, NB{});
    };

    f32x16 acc[I][J];
#pragma unroll
    for (int i = 0; i < I; ++i)
#pragma unroll
        for (int j = 0; j < J; ++j) acc[i][j] = f32x16{};
    // k chunks kc0 .. nk-1: where op(A) is triangular, the chunks of its nonzero part only
    int kc0 = 0, nk = (K + kTK - 1) / kTK;
    if (tri == kGemmLowerA) nk = min(nk, (m0 + BM + kTK - 1) / kTK);
    if (tri == kGemmUpperA) kc0 = min(nk, m0 / kTK);
    const int kh = lane >> 5;
    const int rl = lane & 31;
    if (kc0 < nk) {
        load(kc0 * kTK);
        store(kc0 & 1);
    }
    __syncthreads();
    for (int kc = kc0; kc < nk; ++kc) {
        const int buf = kc & 1;
        if (kc + 1 < nk) load((kc + 1) * kTK);
        float a[I][8], b[J][8];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int i = 0; i < I; ++i) {
                const int ar = 32 * (I * wm + i) + rl;
                const f32x4 x = *reinterpret_cast<const f32x4*>(&As[buf][op_off(ar, 8 * kh + 4 * h)]);
#pragma unroll
                for (int e = 0; e < 4; ++e) a[i][4 * h + e] = x[e];
            }
#pragma unroll
            for (int j = 0; j < J; ++j) {
                const int br = 32 * (J * wn + j) + rl;
                const f32x4 y = *reinterpret_cast<const f32x4*>(&Bs[buf][op_off(br, 8 * kh + 4 * h)]);
#pragma unroll
                for (int e = 0; e < 4; ++e) b[j][4 * h + e] = y[e];
            }
        }
#pragma unroll
        for (int st = 0; st < kTK / 2; ++st)
#pragma unroll
            for (int i = 0; i < I; ++i)
#pragma unroll
                for (int j = 0; j < J; ++j) acc[i][j] = mfma_32x32x2_f32(a[i][st], b[j][st], acc[i][j]);
        if (kc + 1 < nk) store(buf ^ 1);
        __syncthreads();
    }

#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int col = n0 + 32 * (J * wn + j) + rl;
        if (col >= N) continue;
#pragma unroll
        for (int i = 0; i < I; ++i) {
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int row = m0 + 32 * (I * wm + i) + acc_row(v, kh);
                if (row < M) {
                    float* p = Cb + static_cast<long long>(row) * N + col;
                    *p = beta == 0.0f ? alpha * acc[i][j][v] : fmaf(alpha, acc[i][j][v], beta * *p);
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------------------
// Copy-pipelined kernel (K % 16 == 0, 16-byte loads).  The operand tiles of a k chunk go
// HBM -> LDS with global_load_lds_dwordx4, S chunks in flight, so the HBM latency of a chunk
// is covered by the MFMA work of the S - 1 chunks before it instead of one.  A copy writes
// 1 KB of LDS contiguously (lane i: bytes 16i ..), so the layout is chosen by which global
// 16 bytes each lane fetches:
//   * k-contiguous operand (row form): row r of the tile holds its 16 k as four 16-byte
//     chunks, chunk c at slot c ^ ((r / 4) % 4); lane (r, kh) reads chunks 2kh, 2kh + 1
//     (k = 8kh .. 8kh + 7) with two 16-byte reads, 16 rows of a read on distinct banks;
//   * row-contiguous operand (k form): k-row k of the tile holds R floats, 16-byte chunk c
//     at slot c ^ (8 * ((k / 8) % 2)); lane (r, kh) reads k = 8kh + s at step s, 4 bytes,
//     the two lane halves on the two halves of the banks.
// MFMA step s contracts k = s (lanes 0-31) and k = 8 + s (lanes 32-63) of the chunk.
// Rows past M (or N) are fetched from the last valid row (or 4-column group): they only feed
// outputs that are not stored.
// ---------------------------------------------------------------------------------------
template <bool KC, int R>
__device__ __forceinline__ void dma_operand(const float* base, int ld, int r0, int rlim, int k0,
                                            uint32_t lds, int wave, int lane) {
    constexpr int kInst = R * kTK * 4 / 1024;
    static_assert(kInst % (kThreads / kWave) == 0, "copies split evenly over the waves");
#pragma unroll
    for (int i = wave; i < kInst; i += kThreads / kWave) {
        const int p = i * kWave + lane;  // 16-byte slot of the tile
        uint32_t voff;
        if constexpr (KC) {
            const int r = p >> 2;
            const int c = (p & 3) ^ ((r >> 2) & 3);
            const int rr = min(r0 + r, rlim - 1);
            voff = static_cast<uint32_t>((static_cast<long long>(rr) * ld + k0 + 4 * c) * 4);
        } else {
            constexpr int kCpr = R / 4;  // chunks per k-row
            const int k = p / kCpr;
            const int c = (p % kCpr) ^ (((k >> 3) & 1) << 3);
            const int rr = min(r0 + 4 * c, rlim - 4);
            voff = static_cast<uint32_t>((static_cast<long long>(k0 + k) * ld + rr) * 4);
        }
        dma_dwordx4(base, lds + static_cast<uint32_t>(i) * 1024u, voff);
    }
}

// Lane (rl, kh)'s eight k of 32-row block `blk` of an operand tile at LDS float address t:
// x[s] = element (32 blk + rl, 8kh + s).
template <bool KC, int R>
__device__ __forceinline__ void read_operand(const float* t, int blk, int rl, int kh,
                                             float (&x)[8]) {
    const int r = 32 * blk + rl;
    if constexpr (KC) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int c = 2 * kh + h;
            const f32x4 v = *reinterpret_cast<const f32x4*>(t + r * kTK + ((c ^ ((r >> 2) & 3)) << 2));
#pragma unroll
            for (int e = 0; e < 4; ++e) x[4 * h + e] = v[e];
        }
    } else {
        const int rs = r ^ (kh << 5);  // chunk slot swizzle 8 * kh, in floats
#pragma unroll
        for (int s = 0; s < 8; ++s) x[s] = t[(8 * kh + s) * R + rs];
    }
}

// Jobs: a batch's jobs are its (row tile, column tile) pairs, row-major, except that
//   * TRI (ATTN lower-triangular output, square tiles): only the tiles at or below the
//     diagonal, (0,0), (1,0), (1,1), (2,0), ...;
//   * PAIR (for a triangular A): job (p, nt) computes row tiles tiles_m - 1 - p and p one
//     after the other (p < tiles_m / 2, and the middle row tile of an odd count alone), so
//     that every job covers the same number of k chunks.
// The dispatcher deals workgroups to the 8 XCDs round-robin; workgroup w runs job
// (w % 8) * per + w / 8 (per = the grid / 8), so each XCD works through one contiguous
// eighth of the jobs and its L2 serves the operand tiles those jobs share.
template <bool TA, bool TB, int WM, int I, int J, int S, bool PAIR, bool TRI>
__global__ __launch_bounds__(kThreads) void bgemm_f32_dma_kernel(
    const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, int M,
    int N, int K, long long sA, long long sB, long long sC, float alpha, float beta,
    int tiles_m, int tiles_n, int tri, long long jobs) {
    constexpr int WN = 4 / WM;
    constexpr int BM = 32 * I * WM, BN = 32 * J * WN;
    constexpr int kA = BM * kTK, kB = BN * kTK;  // floats of each operand per stage
    constexpr bool KA = !TA, KB = TB;            // k-contiguous in memory
    __shared__ __attribute__((aligned(1024))) float lds[S][kA + kB];
    const long long per = gridDim.x / kXcds;
    const long long job = (blockIdx.x % kXcds) * per + blockIdx.x / kXcds;
    if (job >= jobs) return;
    const int rows = PAIR ? (tiles_m + 1) / 2 : tiles_m;
    const long long tiles = TRI ? static_cast<long long>(tiles_m) * (tiles_m + 1) / 2
                                : static_cast<long long>(rows) * tiles_n;
    const long long batch = job / tiles;
    const int t = static_cast<int>(job - batch * tiles);
    int p, nt;
    if constexpr (TRI) {  // t = p (p + 1) / 2 + nt, nt <= p
        p = static_cast<int>((sqrtf(8.0f * t + 1.0f) - 1.0f) * 0.5f);
        while (p * (p + 1) / 2 > t) --p;
        while ((p + 1) * (p + 2) / 2 <= t) ++p;
        nt = t - p * (p + 1) / 2;
    } else {
        p = t / tiles_n;
        nt = t % tiles_n;
    }
    const int n0 = nt * BN;
    const float* Ab = A + batch * sA;
    const float* Bb = B + batch * sB;
    float* Cb = C + batch * sC;
    const int lda = TA ? M : K;
    const int ldb = TB ? K : N;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
    const int wm = wave % WM, wn = wave / WM;
    const int kh = lane >> 5, rl = lane & 31;
    const uint32_t lds0 = lds_addr(&lds[0][0]);
    constexpr uint32_t kStageBytes = (kA + kB) * 4;
    // copy instructions per wave per chunk
    constexpr int kPerWave = (kA + kB) * 4 / 1024 / (kThreads / kWave);

    const int nparts = PAIR && 2 * p + 1 != tiles_m ? 2 : 1;
    for (int part = 0; part < nparts; ++part) {
        const int mt = PAIR ? (part == 0 ? tiles_m - 1 - p : p) : p;
        const int m0 = mt * BM;
        if (tri == kGemmLowerOut && n0 > m0 + BM - 1) continue;  // wholly above the diagonal
        int kc0 = 0, nk = K / kTK;
        if (tri == kGemmLowerA) nk = min(nk, (m0 + BM + kTK - 1) / kTK);
        if (tri == kGemmUpperA) kc0 = min(nk, m0 / kTK);
        auto issue = [&](int kc) {
            const uint32_t st = lds0 + static_cast<uint32_t>((kc - kc0) % S) * kStageBytes;
            dma_operand<KA, BM>(Ab, lda, m0, M, kc * kTK, st, wave, lane);
            dma_operand<KB, BN>(Bb, ldb, n0, N, kc * kTK, st + kA * 4, wave, lane);
        };

        f32x16 acc[I][J];
#pragma unroll
        for (int i = 0; i < I; ++i)
#pragma unroll
            for (int j = 0; j < J; ++j) acc[i][j] = f32x16{};
        if (part > 0) __syncthreads();  // the previous part's last chunk is no longer read
#pragma unroll
        for (int s = 0; s < S - 1; ++s)
            if (kc0 + s < nk) issue(kc0 + s);
        for (int kc = kc0; kc < nk; ++kc) {
            // chunks issued after kc: kc + 1 .. min(nk - 1, kc + S - 2); the first wait of a
            // part also covers the previous part's stores, so it waits for everything
            if (kc == kc0) wait_vm<0>();
            else wait_vm_at_most(min(nk - 1 - kc, S - 2) * kPerWave);
            __syncthreads();  // chunk kc landed for every wave; chunk kc - 1 is no longer read
            if (kc + S - 1 < nk) issue(kc + S - 1);
            const float* st = &lds[(kc - kc0) % S][0];
            float a[I][8], b[J][8];
#pragma unroll
            for (int i = 0; i < I; ++i) read_operand<KA, BM>(st, I * wm + i, rl, kh, a[i]);
#pragma unroll
            for (int j = 0; j < J; ++j) read_operand<KB, BN>(st + kA, J * wn + j, rl, kh, b[j]);
#pragma unroll
            for (int s = 0; s < 8; ++s)
#pragma unroll
                for (int i = 0; i < I; ++i)
#pragma unroll
                    for (int j = 0; j < J; ++j)
                        acc[i][j] = mfma_32x32x2_f32(a[i][s], b[j][s], acc[i][j]);
        }

#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int col = n0 + 32 * (J * wn + j) + rl;
            if (col >= N) continue;
#pragma unroll
            for (int i = 0; i < I; ++i) {
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int row = m0 + 32 * (I * wm + i) + acc_row(v, kh);
                    if (row < M) {
                        float* q = Cb + static_cast<long long>(row) * N + col;
                        *q = beta == 0.0f ? alpha * acc[i][j][v]
                                          : fmaf(alpha, acc[i][j][v], beta * *q);
                    }
                }
            }
        }
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <bool TA, bool TB, int WM, int I, int J, int S, bool PAIR, bool TRI = false>
void launch_dma(const float* A, const float* B, float* C, int M, int N, int K, long long sA,
                long long sB, long long sC, int batch, float alpha, float beta,
                hipStream_t stream, GemmTri tri) {
    constexpr int BM = 32 * I * WM, BN = 32 * J * (4 / WM);
    const int tm = (M + BM - 1) / BM, tn = (N + BN - 1) / BN;
    const long long tiles = TRI ? static_cast<long long>(tm) * (tm + 1) / 2
                                : static_cast<long long>(PAIR ? (tm + 1) / 2 : tm) * tn;
    const long long jobs = tiles * batch;
    const long long per = (jobs + kXcds - 1) / kXcds;
    hipLaunchKernelGGL((bgemm_f32_dma_kernel<TA, TB, WM, I, J, S, PAIR, TRI>),
                       dim3(static_cast<unsigned>(per * kXcds)), dim3(kThreads), 0, stream, A, B,
                       C, M, N, K, sA, sB, sC, alpha, beta, tm, tn, static_cast<int>(tri), jobs);
}

template <bool TA, bool TB>
void launch_tiled(const float* A, const float* B, float* C, int M, int N, int K, long long sA,
                  long long sB, long long sC, int batch, float alpha, float beta,
                  hipStream_t stream, GemmTri tri) {
    const dim3 b(kThreads);
    // the copy-pipelined kernel addresses each batch's operands with 32-bit byte offsets
    const long long lim = 0xffffffffLL;
    if (K % kTK == 0 && 4LL * M * K <= lim && 4LL * K * N <= lim) {
        if (N > 64 && tri == kGemmLowerOut)  // 128 x 128 tiles at or below the diagonal
            // two stages: at config 2 (K = 64, four chunks per tile) QK^T 110 -> 101 us
            launch_dma<TA, TB, 2, 2, 2, 2, false, true>(A, B, C, M, N, K, sA, sB, sC, batch,
                                                        alpha, beta, stream, tri);
        else if (N > 64)  // 128 x 128: each wave 64 x 64
            launch_dma<TA, TB, 2, 2, 2, 3, false>(A, B, C, M, N, K, sA, sB, sC, batch, alpha,
                                                  beta, stream, tri);
        else if (tri == kGemmLowerA || tri == kGemmUpperA)  // 64 x 64 row tiles in pairs
            launch_dma<TA, TB, 2, 1, 1, 4, true>(A, B, C, M, N, K, sA, sB, sC, batch, alpha,
                                                 beta, stream, tri);
        else  // 128 x 64: each wave 32 x 64
            launch_dma<TA, TB, 4, 1, 2, 3, false>(A, B, C, M, N, K, sA, sB, sC, batch, alpha,
                                                  beta, stream, tri);
        return;
    }
    if (N <= 64) {  // 128 x 64: each wave 32 x 64
        const int tm = (M + 127) / 128, tn = (N + 63) / 64;
        hipLaunchKernelGGL((bgemm_f32_tiled_kernel<TA, TB, 4, 1, 2>),
                           dim3(static_cast<unsigned>(static_cast<long long>(tm) * tn * batch)), b,
                           0, stream, A, B, C, M, N, K, sA, sB, sC, alpha, beta, tm, tn,
                           static_cast<int>(tri));
    } else {  // 128 x 128: each wave 64 x 64
        const int tm = (M + 127) / 128, tn = (N + 127) / 128;
        hipLaunchKernelGGL((bgemm_f32_tiled_kernel<TA, TB, 2, 2, 2>),
                           dim3(static_cast<unsigned>(static_cast<long long>(tm) * tn * batch)), b,
                           0, stream, A, B, C, M, N, K, sA, sB, sC, alpha, beta, tm, tn,
                           static_cast<int>(tri));
    }
}

}  // namespace

void launch_batched_gemm_f32(const float* A, const float* B, float* C, int M, int N, int K,
                             long long sA, long long sB, long long sC, int batch, bool transA,
                             bool transB, float alpha, float beta, hipStream_t stream,
                             GemmTri tri) {
    // 16-byte loads need the contiguous dimension of each operand (K or M for A, N or K for
    // B) a multiple of 4 and 16-byte aligned bases and batch strides
    const bool vec = ((transA ? M : K) % 4 == 0) && ((transB ? K : N) % 4 == 0) &&
                     sA % 4 == 0 && sB % 4 == 0 && aligned16(A) && aligned16(B);
    if (vec) {
        if (transA) {
            if (transB)
                launch_tiled<true, true>(A, B, C, M, N, K, sA, sB, sC, batch, alpha, beta, stream,
                                         tri);
            else
                launch_tiled<true, false>(A, B, C, M, N, K, sA, sB, sC, batch, alpha, beta, stream,
                                          tri);
        } else {
            if (transB)
                launch_tiled<false, true>(A, B, C, M, N, K, sA, sB, sC, batch, alpha, beta, stream,
                                          tri);
            else
                launch_tiled<false, false>(A, B, C, M, N, K, sA, sB, sC, batch, alpha, beta,
                                           stream, tri);
        }
        return;
    }
    // the scalar kernel skips the zero part of a triangular A as the others do (so no kernel
    // reads a lower-triangular A past the end of the 128-column block holding the diagonal)
    // and writes every output
    const int tiles_m = (M + kBM - 1) / kBM;
    const int tiles_n = (N + kBN - 1) / kBN;
    const long long grid = static_cast<long long>(tiles_m) * tiles_n * batch;
    const dim3 g(static_cast<unsigned>(grid)), b(kThreads);
    const int tr = static_cast<int>(tri);
    if (transA) {
        if (transB)
            hipLaunchKernelGGL((bgemm_f32_kernel<true, true>), g, b, 0, stream, A, B, C, M, N,
                               K, sA, sB, sC, alpha, beta, tiles_m, tiles_n, tr);
        else
            hipLaunchKernelGGL((bgemm_f32_kernel<true, false>), g, b, 0, stream, A, B, C, M, N,
                               K, sA, sB, sC, alpha, beta, tiles_m, tiles_n, tr);
    } else {
        if (transB)
            hipLaunchKernelGGL((bgemm_f32_kernel<false, true>), g, b, 0, stream, A, B, C, M, N,
                               K, sA, sB, sC, alpha, beta, tiles_m, tiles_n, tr);
        else
            hipLaunchKernelGGL((bgemm_f32_kernel<false, false>), g, b, 0, stream, A, B, C, M,
                               N, K, sA, sB, sC, alpha, beta, tiles_m, tiles_n, tr);
    }
}

}  // namespace tcamd
