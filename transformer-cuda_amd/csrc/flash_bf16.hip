// flash_bf16.hip - tiled causal attention backward, bf16 fast path, on
// v_mfma_f32_32x32x16_bf16 with fp32 accumulation (the forward is in flash_bf16_fwd.hip).
//
// Algorithm: the reference's analytical backward (src/kernels/attention.cu:626-955) in the
// split form of the fp32 path: stage 1 (query-parallel) writes D = rowsum(dO * O) and dQ,
// stage 2 (key-parallel) dK and dV, both recomputing P = 2^(s*c - lse2) from the forward's
// statistics (lse2 = m*log2 e + log2 l, the log2-domain log-sum-exp).  P and dS are rounded
// to bf16 as MFMA operands; dQ/dK/dV are rounded once, at the store.
//
// Both stages use the forward's staging: 64-row tiles copied HBM -> LDS with
// global_load_lds_dwordx4 into XOR-swizzled rows, double buffered and shared by the 4 waves
// of a workgroup.  A product that contracts over the head dimension reads its A operand as
// 16-byte row reads of a tile and its B operand from VGPRs; a product that contracts over
// the sequence reads its A operand with ds_read_tr16_b64 from the same row-major tile and
// takes its B operand (P or dS, rounded to bf16) straight from the accumulator of the
// score product, whose rows are the contracted positions.
//
// Stage 1, per 32-key half tile and 32-query sub-block (d = 64: 12 MFMAs):
//   S^T  = K Q^T      A = K rows,  B = Q (VGPRs)
//   dP^T = V dO^T     A = V rows,  B = dO (VGPRs)
//   dS^T = P^T o (dP^T - D)        lane l holds query l%32: lse2 and D are per lane
//   dQ^T += K^T dS^T  A = K^T (transposing reads of the K tile), B = dS^T
// A workgroup owns 256 queries (d <= 64; wave w: sub-blocks w and 7-w, as the forward) or
// 128 (d = 128, one sub-block per wave, for registers).
//
// Stage 2, per 32-query half tile and a wave's 32 keys (d = 64: 18 MFMAs):
//   S  = Q K^T        A = Q rows,  B = K (VGPRs)
//   dP = dO V^T       A = dO rows, B = V (VGPRs)
//   dS = P o (dP - D)              -lse2 and -D enter S and dP as one more contraction step
//                                  over a per-row (hi, lo) bf16 chunk (see dkdv_scores); K is
//                                  held pre-multiplied by c = scale*log2 e, so P = 2^S
//                                  needs no per-element multiply
//   dV^T += dO^T P    A = dO^T (transposing reads), B = P
//   dK^T += Q^T dS    A = Q^T (transposing reads),  B = dS
// A workgroup owns 128 keys; query tiles start at the workgroup's first key, and wave w
// joins at the half tile that holds its first key (the only one it masks).  A wave handles
// both half tiles of a 64-query tile per step, so the MFMAs of one overlap the softmax
// arithmetic of the other.
#include <math.h>

#include <type_traits>

#include "bf16_tile.hpp"
#include "device_common.hpp"
#include "launch.hpp"

namespace tcamd {
namespace {

using namespace bf16t;

// K and V tiles of stage 1 (same shape as the forward's).
template <int D>
struct KvSmem {
    uint16_t k[2][Swz<D>::kBytes / 2];
    uint16_t v[2][Swz<D>::kBytes / 2];
};

// Q and dO tiles of stage 2, each with an extra 8-element column chunk per row that carries
// the row's statistic (see dkdv_scores).
template <int D>
struct QgSmem {
    uint16_t q[2][Swz<D>::kBytes / 2];
    uint16_t g[2][Swz<D>::kBytes / 2];
    uint16_t qx[2][kRowTile * 8];  // row r: (-lse2)_hi, (-lse2)_lo, 0 x 6
    uint16_t gx[2][kRowTile * 8];  // row r: (-D)_hi, (-D)_lo, 0 x 6
};

// x as the bf16 pair (hi, lo), hi + lo = x to ~2^-16 relative, packed into one dword.
__device__ __forceinline__ uint32_t split_bf16x2(float x) {
    const uint16_t hi = f32_to_bf16_bits(x);
    const uint16_t lo = f32_to_bf16_bits(x - bf16_bits_to_f32(hi));
    return static_cast<uint32_t>(hi) | (static_cast<uint32_t>(lo) << 16);
}

// The B or A operand (1, 1, 0, ...) of a contraction step that adds a per-row statistic
// (hi, lo) to a product: lanes of k-group 1 hold zeros.
__device__ __forceinline__ bf16x8 ones_pair(int half) {
    bf16x8 one = bf16x8{};
    if (half == 0) {
        one[0] = static_cast<__bf16>(1.0f);
        one[1] = static_cast<__bf16>(1.0f);
    }
    return one;
}

// The statistic chunk (x_hi, x_lo, 0, ...) of a lane's row (zeros in k-group 1).
__device__ __forceinline__ bf16x8 stat_chunk(float x, int half) {
    u16x8 v = u16x8{};
    if (half == 0) {
        const uint32_t p = split_bf16x2(x);
        v[0] = static_cast<uint16_t>(p);
        v[1] = static_cast<uint16_t>(p >> 16);
    }
    return __builtin_bit_cast(bf16x8, v);
}

// ---------------------------------------------------------------------------------------
// Stage 1: D and dQ.
// ---------------------------------------------------------------------------------------

// One 32-query sub-block of a wave.
template <int D>
struct DqSub {
    bf16x8 q[D / 16];    // c * Q row of query col (B operand over d)
    bf16x8 g[D / 16];    // dO row
    bf16x8 xs, xd;       // statistic chunks: -lse2 (-1e30 for padded queries: P = 0), -D
    f32x16 acc[D / 32];  // dQ^T
};

// qh: this head's q (rows xrs apart); oh, gh: its o and dO (rows ors apart).  Q is held
// pre-multiplied by c = scale*log2 e and rounded to bf16 (one extra rounding, ~2^-9
// relative per element), so that the scores come out in the log2 domain.
template <int D>
__device__ __forceinline__ void dq_init(DqSub<D>& sb, const uint16_t* __restrict__ qh,
                                        const uint16_t* __restrict__ oh,
                                        const uint16_t* __restrict__ gh,
                                        const float* __restrict__ m, const float* __restrict__ l,
                                        float* __restrict__ Dws, int xrs, int ors,
                                        size_t stat_off, int qi, int T, int half, float c) {
    load_rowop<D>(sb.q, qh, qi, T, half, xrs);
    load_rowop<D>(sb.g, gh, qi, T, half, ors);
    bf16x8 orow[D / 16];
    load_rowop<D>(orow, oh, qi, T, half, ors);
    float part = 0.0f;
#pragma unroll
    for (int j = 0; j < D / 16; ++j) {
#pragma unroll
        for (int e = 0; e < 8; ++e)
            part = fmaf(static_cast<float>(sb.g[j][e]), static_cast<float>(orow[j][e]), part);
    }
#pragma unroll
    for (int j = 0; j < D / 16; ++j) {
#pragma unroll
        for (int e = 0; e < 8; ++e) sb.q[j][e] = static_cast<__bf16>(static_cast<float>(sb.q[j][e]) * c);
    }
    const float dlt = xhalf_sum(part);
    float nl = -1e30f;
    if (qi < T) {
        if (half == 0) Dws[stat_off + qi] = dlt;
        nl = -(m[stat_off + qi] * kLog2e + log2f(l[stat_off + qi]));
    }
    sb.xs = stat_chunk(nl, half);
    sb.xd = stat_chunk(-dlt, half);
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) sb.acc[dt] = f32x16{};
}

// s = S'^T = K (cQ)^T - lse2, dp = dP'^T = V dO^T - D of keys kb.. (rows) x queries qj + col
// (columns) -> dS^T = 2^s o dp as the two B operands of dQ^T += K^T dS^T.  Keys past the
// query get P = 0.
__device__ __forceinline__ void dq_ds(f32x16& s, const f32x16& dp, bf16x8 (&db)[2], int kb,
                                      int qj, int col, int half) {
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = exp2_fast(s[r]);
    if (kb + 31 > qj) {  // the half tile crosses the diagonal of this sub-block
#pragma unroll
        for (int r = 0; r < 16; ++r)
            if (kb + acc_row(r, half) > qj + col) s[r] = 0.0f;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] *= dp[r];
    db[0] = pack_b(s, 0);
    db[1] = pack_b(s, 1);
}

// One 32-key half tile for sub-block 1, and sub-block 0 too when BOTH.  ka/va: this lane's
// row-read addresses in the K / V tile; kta: transposing-read addresses in the K tile.
// -lse2 and -D enter S^T and dP^T as one more contraction step: the A operand `one`
// (1, 1, 0, ...) times the sub-block's statistic chunks (hi, lo, 0, ...).
template <int D, bool BOTH>
__device__ __forceinline__ void dq_half(int kb, const uint32_t (&ka)[D / 16],
                                        const uint32_t (&va)[D / 16],
                                        const uint32_t (&kta)[D / 32], const bf16x8& one,
                                        DqSub<D>& sb0, DqSub<D>& sb1, int qj0, int qj1, int col,
                                        int half) {
    f32x16 s0, s1, p0, p1;
    s1 = mfma_32x32x16_bf16(one, sb1.xs, f32x16{});
    if constexpr (BOTH) s0 = mfma_32x32x16_bf16(one, sb0.xs, f32x16{});
#pragma unroll
    for (int st = 0; st < D / 16; ++st) {
        const bf16x8 a = lds_b128(ka[st]);
        s1 = mfma_32x32x16_bf16(a, sb1.q[st], s1);
        if constexpr (BOTH) s0 = mfma_32x32x16_bf16(a, sb0.q[st], s0);
    }
    p1 = mfma_32x32x16_bf16(one, sb1.xd, f32x16{});
    if constexpr (BOTH) p0 = mfma_32x32x16_bf16(one, sb0.xd, f32x16{});
#pragma unroll
    for (int st = 0; st < D / 16; ++st) {
        const bf16x8 a = lds_b128(va[st]);
        p1 = mfma_32x32x16_bf16(a, sb1.g[st], p1);
        if constexpr (BOTH) p0 = mfma_32x32x16_bf16(a, sb0.g[st], p0);
    }
    bf16x8 d0[2], d1[2];
    dq_ds(s1, p1, d1, kb, qj1, col, half);
    if constexpr (BOTH) dq_ds(s0, p0, d0, kb, qj0, col, half);
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const bf16x8 a = lds_tr(kta[dt] + u * Swz<D>::rows(16), Swz<D>::rows(8));
            sb1.acc[dt] = mfma_32x32x16_bf16(a, d1[u], sb1.acc[dt]);
            if constexpr (BOTH) sb0.acc[dt] = mfma_32x32x16_bf16(a, d0[u], sb0.acc[dt]);
        }
    }
}

// NSUB = 2: 256 queries per workgroup, wave w owns sub-blocks w (0) and 7-w (1).
// NSUB = 1: 128 queries per workgroup, wave w owns sub-block w (1).
template <int D, int NSUB>
__global__ __launch_bounds__(kWave* kWaves) void flash_bwd_dq_bf16_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const uint16_t* __restrict__ o,
    const uint16_t* __restrict__ dO, const float* __restrict__ m, const float* __restrict__ l,
    uint16_t* __restrict__ dq, float* __restrict__ Dws, int BH, int T, float scale, int nblk,
    HeadView xv, HeadView ov, HeadView gv) {
    using S = Swz<D>;
    constexpr int kBlock = kWaves * NSUB * kSub;
    __shared__ __attribute__((aligned(1024))) KvSmem<D> sm;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int lane = threadIdx.x & (kWave - 1);
    const int col = lane & 31;
    const int half = lane >> 5;
    int bh, blk;
    map_block(blockIdx.x, BH, nblk, true, bh, blk);
    const int q0 = blk * kBlock;
    const int qj0 = q0 + kSub * wave;
    const int qj1 = NSUB == 2 ? q0 + kSub * (2 * kWaves - 1 - wave) : qj0;
    const size_t xoff = xv.off(bh), ooff = ov.off(bh), goff = gv.off(bh);
    const int xrs = xv.row, ors = ov.row, grs = gv.row;
    const size_t stat_off = static_cast<size_t>(bh) * T;
    const uint16_t* kh = k + xoff;
    const uint16_t* vh = v + xoff;
    const float c = scale * kLog2e;

    const int kend = min(T, q0 + kBlock);
    const int ntile = (kend + kRowTile - 1) / kRowTile;
    const uint32_t k_lds = lds_addr(sm.k[0]);
    const uint32_t v_lds = lds_addr(sm.v[0]);
    dma_tile<D>(kh, 0, T, k_lds, wave, lane, xrs);
    dma_tile<D>(vh, 0, T, v_lds, wave, lane, xrs);

    DqSub<D> sb0, sb1;
    dq_init<D>(sb1, q + xoff, o + ooff, dO + ooff, m, l, Dws, xrs, ors, stat_off, qj1 + col, T,
               half, c);
    if constexpr (NSUB == 2)
        dq_init<D>(sb0, q + xoff, o + ooff, dO + ooff, m, l, Dws, xrs, ors, stat_off, qj0 + col,
                   T, half, c);
    const bf16x8 one = ones_pair(half);

    uint32_t roff[D / 16], troff[D / 32];
    lane_offsets<D>(lane, roff, troff);

    const int nhalf_t = (T + 31) / 32;
    const int hA = NSUB == 2 ? min(qj0 / 32 + 1, nhalf_t) : 0;
    const int hB = min(qj1 / 32 + 1, nhalf_t);
    const int hend = 2 * ntile;
    uint32_t ka[D / 16], va[D / 16], kta[D / 32];
    auto tile_sync = [&](int hh) {
        const int kt = hh >> 1;
        if ((hh & 1) == 0) {
            wait_vm<0>();     // this wave's copies of tile kt landed ...
            __syncthreads();  // ... and every wave's; tile kt-1 is no longer read by anyone
            if (kt + 1 < ntile) {
                const uint32_t nbuf = static_cast<uint32_t>((kt + 1) & 1) * S::kBytes;
                dma_tile<D>(kh, (kt + 1) * kRowTile, T, k_lds + nbuf, wave, lane, xrs);
                dma_tile<D>(vh, (kt + 1) * kRowTile, T, v_lds + nbuf, wave, lane, xrs);
            }
        }
        const uint32_t base = static_cast<uint32_t>(kt & 1) * S::kBytes +
                              static_cast<uint32_t>(hh & 1) * S::rows(32);
#pragma unroll
        for (int st = 0; st < D / 16; ++st) {
            ka[st] = k_lds + base + roff[st];
            va[st] = v_lds + base + roff[st];
        }
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) kta[dt] = k_lds + base + troff[dt];
    };
    int hh = 0;
    for (; hh < hA; ++hh) {
        tile_sync(hh);
        dq_half<D, true>(32 * hh, ka, va, kta, one, sb0, sb1, qj0, qj1, col, half);
    }
    for (; hh < hB; ++hh) {
        tile_sync(hh);
        dq_half<D, false>(32 * hh, ka, va, kta, one, sb0, sb1, qj0, qj1, col, half);
    }
    for (; hh < hend; ++hh) tile_sync(hh);

    if (qj1 + col < T) store_row<D>(dq + goff, qj1 + col, half, sb1.acc, scale, grs);
    if constexpr (NSUB == 2)
        if (qj0 + col < T) store_row<D>(dq + goff, qj0 + col, half, sb0.acc, scale, grs);
}

// ---------------------------------------------------------------------------------------
// Stage 2: dK, dV.
// ---------------------------------------------------------------------------------------

// Per-lane operands of one 32-query half tile of stage 2.
template <int D>
struct HalfAddr {
    uint32_t q[D / 16], g[D / 16];    // row reads, chunk step st
    uint32_t qt[D / 32], gt[D / 32];  // transposing reads, head-dim tile dt
    uint32_t qx, gx;                  // statistic chunks of row col
};

// S' = Q (cK)^T - lse2 and dP' = dO V^T - D of one half tile.  The statistics ride in the
// products: a fifth 16-wide contraction step multiplies the row's chunk (hi, lo, 0, ...)
// by the B operand `one` = (1, 1, 0, ...) (lanes of k-group 1 hold zeros), so that
// 2^S' = P and P o dP' = dS need no per-row values in VGPRs.
template <int D>
__device__ __forceinline__ void dkdv_scores(const HalfAddr<D>& a, const bf16x8 (&kr)[D / 16],
                                            const bf16x8 (&vr)[D / 16], const bf16x8& one,
                                            f32x16& s, f32x16& dp) {
    s = mfma_32x32x16_bf16(lds_b128(a.qx), one, f32x16{});
#pragma unroll
    for (int st = 0; st < D / 16; ++st) s = mfma_32x32x16_bf16(lds_b128(a.q[st]), kr[st], s);
    dp = mfma_32x32x16_bf16(lds_b128(a.gx), one, f32x16{});
#pragma unroll
    for (int st = 0; st < D / 16; ++st) dp = mfma_32x32x16_bf16(lds_b128(a.g[st]), vr[st], dp);
}

// P = 2^S' (0 where the query precedes the key, on the diagonal half tile) and
// dS = P o dP'; dV^T += dO^T P, dK^T += Q^T dS.
template <int D, bool MASK>
__device__ __forceinline__ void dkdv_update(const HalfAddr<D>& a, f32x16& s, const f32x16& dp,
                                            f32x16 (&dk_acc)[D / 32],
                                            f32x16 (&dv_acc)[D / 32], int qb, int kj,
                                            int half) {
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = exp2_fast(s[r]);
    if constexpr (MASK) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
            if (qb + acc_row(r, half) < kj) s[r] = 0.0f;
    }
    const bf16x8 pb[2] = {pack_b(s, 0), pack_b(s, 1)};
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] *= dp[r];
    const bf16x8 db[2] = {pack_b(s, 0), pack_b(s, 1)};
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            dv_acc[dt] =
                mfma_32x32x16_bf16(lds_tr(a.gt[dt] + u * Swz<D>::rows(16), Swz<D>::rows(8)), pb[u], dv_acc[dt]);
            dk_acc[dt] =
                mfma_32x32x16_bf16(lds_tr(a.qt[dt] + u * Swz<D>::rows(16), Swz<D>::rows(8)), db[u], dk_acc[dt]);
        }
    }
}

// NW waves per workgroup; wave w owns keys k0 + 32w ...
template <int D, int NW>
__global__ __launch_bounds__(kWave* NW) void flash_bwd_dkdv_bf16_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const uint16_t* __restrict__ dO,
    const float* __restrict__ m, const float* __restrict__ l, const float* __restrict__ Dws,
    uint16_t* __restrict__ dk, uint16_t* __restrict__ dv, int BH, int T, float scale,
    int nblk, HeadView xv, HeadView ov, HeadView gv) {
    using S = Swz<D>;
    constexpr int kBlock = NW * kSub;  // keys per workgroup
    __shared__ __attribute__((aligned(1024))) QgSmem<D> sm;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int lane = threadIdx.x & (kWave - 1);
    const int col = lane & 31;
    const int half = lane >> 5;
    int bh, blk;
    map_block(blockIdx.x, BH, nblk, false, bh, blk);  // block 0 sees every query
    const int k0 = blk * kBlock;
    const int kw = k0 + kSub * wave;
    const int kj = kw + col;
    const size_t xoff = xv.off(bh), ooff = ov.off(bh), goff = gv.off(bh);
    const int xrs = xv.row, ors = ov.row, grs = gv.row;
    const size_t stat_off = static_cast<size_t>(bh) * T;
    const uint16_t* qh = q + xoff;
    const uint16_t* gh = dO + ooff;
    const float c = scale * kLog2e;

    const int t0 = k0 / kRowTile;
    const int ntile = (T + kRowTile - 1) / kRowTile;
    const uint32_t q_lds = lds_addr(sm.q[0]);
    const uint32_t g_lds = lds_addr(sm.g[0]);
    const uint32_t qx_lds = lds_addr(sm.qx[0]);
    const uint32_t gx_lds = lds_addr(sm.gx[0]);
    dma_tile<D, NW>(qh, t0 * kRowTile, T, q_lds, wave, lane, xrs);
    dma_tile<D, NW>(gh, t0 * kRowTile, T, g_lds, wave, lane, ors);
    // Wave 0 stages the statistics of a tile through VGPRs: lane i holds query 64t + i.
    float st_m = 0.0f, st_l = 1.0f, st_d = 0.0f;
    auto load_stats = [&](int t) {
        const int r = t * kRowTile + lane;
        if (r < T) {
            st_m = m[stat_off + r];
            st_l = l[stat_off + r];
            st_d = Dws[stat_off + r];
        } else {
            st_m = -INFINITY;  // padded query: P = 0 (see tile_sync)
            st_l = 1.0f;
            st_d = 0.0f;
        }
    };
    if (wave == 0) {
        load_stats(t0);
        const u16x8 z = u16x8{};  // the constant zeros of the statistic chunks
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            *reinterpret_cast<u16x8*>(&sm.qx[b][lane * 8]) = z;
            *reinterpret_cast<u16x8*>(&sm.gx[b][lane * 8]) = z;
        }
    }
    const bf16x8 one = ones_pair(half);

    bf16x8 kr[D / 16], vr[D / 16];
    load_rowop<D>(kr, k + xoff, kj, T, half, xrs);
    // c*K rounded to bf16 (one extra rounding, ~2^-9 relative per element; the score error it
    // causes is a random sum over d, ~1e-3 in log2 units for unit-variance inputs)
#pragma unroll
    for (int st = 0; st < D / 16; ++st)
#pragma unroll
        for (int e = 0; e < 8; ++e) kr[st][e] = static_cast<__bf16>(static_cast<float>(kr[st][e]) * c);
    load_rowop<D>(vr, v + xoff, kj, T, half, xrs);
    f32x16 dk_acc[D / 32], dv_acc[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
        dk_acc[dt] = f32x16{};
        dv_acc[dt] = f32x16{};
    }
    uint32_t roff[D / 16], troff[D / 32];
    lane_offsets<D>(lane, roff, troff);
    const uint32_t soff = static_cast<uint32_t>(col * 16);  // statistic chunk of row col

    // Tile kt: wait for its copies, publish its statistics, barrier, start the next copy.
    auto tile_sync = [&](int kt) {
        wait_vm<0>();  // this wave's copies (and statistics loads) of tile kt landed
        if (wave == 0) {  // -lse2 (-1e30 for padded queries: P = 0) and -D as bf16 pairs
            const float nl = st_m == -INFINITY ? -1e30f : -(st_m * kLog2e + log2f(st_l));
            *reinterpret_cast<uint32_t*>(&sm.qx[kt & 1][lane * 8]) = split_bf16x2(nl);
            *reinterpret_cast<uint32_t*>(&sm.gx[kt & 1][lane * 8]) = split_bf16x2(-st_d);
        }
        __syncthreads();  // every wave's copies landed; tile kt-1 is no longer read
        if (kt + 1 < ntile) {
            if (wave == 0) load_stats(kt + 1);
            const uint32_t nbuf = static_cast<uint32_t>((kt + 1) & 1) * S::kBytes;
            dma_tile<D, NW>(qh, (kt + 1) * kRowTile, T, q_lds + nbuf, wave, lane, xrs);
            dma_tile<D, NW>(gh, (kt + 1) * kRowTile, T, g_lds + nbuf, wave, lane, ors);
        }
    };
    // Operand addresses of half tile hh (queries 32*hh ..).
    auto half_addr = [&](int hh) {
        HalfAddr<D> a;
        const int kt = hh >> 1;
        const uint32_t base = static_cast<uint32_t>(kt & 1) * S::kBytes +
                              static_cast<uint32_t>(hh & 1) * S::rows(32);
#pragma unroll
        for (int st = 0; st < D / 16; ++st) {
            a.q[st] = q_lds + base + roff[st];
            a.g[st] = g_lds + base + roff[st];
        }
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) {
            a.qt[dt] = q_lds + base + troff[dt];
            a.gt[dt] = g_lds + base + troff[dt];
        }
        const uint32_t xrow = static_cast<uint32_t>(((kt & 1) * kRowTile + (hh & 1) * 32 + col) * 16);
        a.qx = qx_lds + xrow;
        a.gx = gx_lds + xrow;
        return a;
    };
    // The same with the buffer parity and half a compile-time constant: every address is a
    // lane offset plus an immediate.
    auto half_addr_c = [&](auto buf, auto hsel) {
        HalfAddr<D> a;
        constexpr uint32_t base = static_cast<uint32_t>(decltype(buf)::value) * S::kBytes +
                                  static_cast<uint32_t>(decltype(hsel)::value) * S::rows(32);
        constexpr uint32_t xbase = static_cast<uint32_t>(decltype(buf)::value * kRowTile +
                                                         decltype(hsel)::value * 32) * 16u;
#pragma unroll
        for (int st = 0; st < D / 16; ++st) {
            a.q[st] = roff[st] + (q_lds + base);
            a.g[st] = roff[st] + (g_lds + base);
        }
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) {
            a.qt[dt] = troff[dt] + (q_lds + base);
            a.gt[dt] = troff[dt] + (g_lds + base);
        }
        a.qx = soff + (qx_lds + xbase);
        a.gx = soff + (gx_lds + xbase);
        return a;
    };
    // Both half tiles of tile kt (held in buffer `buf`), no diagonal.
    auto pair_c = [&](int kt, auto buf) {
        const HalfAddr<D> a0 = half_addr_c(buf, std::integral_constant<int, 0>{});
        const HalfAddr<D> a1 = half_addr_c(buf, std::integral_constant<int, 1>{});
        f32x16 s0, dp0, s1, dp1;
        dkdv_scores<D>(a0, kr, vr, one, s0, dp0);
        dkdv_scores<D>(a1, kr, vr, one, s1, dp1);
        dkdv_update<D, false>(a0, s0, dp0, dk_acc, dv_acc, 64 * kt, kj, half);
        dkdv_update<D, false>(a1, s1, dp1, dk_acc, dv_acc, 64 * kt + 32, kj, half);
    };
    // Both half tiles of tile kt; the first is the diagonal one when MASK0.  The score
    // products of the second half tile are issued before the first half tile's softmax.
    auto pair = [&](int kt, auto mask0) {
        const HalfAddr<D> a0 = half_addr(2 * kt), a1 = half_addr(2 * kt + 1);
        f32x16 s0, dp0, s1, dp1;
        dkdv_scores<D>(a0, kr, vr, one, s0, dp0);
        dkdv_scores<D>(a1, kr, vr, one, s1, dp1);
        dkdv_update<D, decltype(mask0)::value>(a0, s0, dp0, dk_acc, dv_acc, 64 * kt, kj, half);
        dkdv_update<D, false>(a1, s1, dp1, dk_acc, dv_acc, 64 * kt + 32, kj, half);
    };

    // Half tiles before hstart (= kw/32, the one holding the wave's first key) hold only
    // queries that precede every key of the wave; a wave whose keys start past T computes
    // nothing.  Every wave takes part in every tile's barrier and copies.
    const int hstart = kw < T ? kw / 32 : 2 * ntile;
    int kt = t0;
    for (; 2 * kt + 1 < hstart; ++kt) tile_sync(kt);
    if (kt < ntile) {  // the tile holding the diagonal half tile
        tile_sync(kt);
        if (hstart & 1) {  // only its second half tile, the diagonal one
            const HalfAddr<D> a1 = half_addr(hstart);
            f32x16 s1, dp1;
            dkdv_scores<D>(a1, kr, vr, one, s1, dp1);
            dkdv_update<D, true>(a1, s1, dp1, dk_acc, dv_acc, 32 * hstart, kj, half);
        } else {
            pair(kt, std::true_type{});
        }
        ++kt;
    }
    // Steady state, unrolled by the buffer parity (tile kt is in buffer kt & 1).
    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;
    if (kt < ntile && (kt & 1)) {
        tile_sync(kt);
        pair_c(kt, B1{});
        ++kt;
    }
    for (; kt + 1 < ntile; kt += 2) {
        tile_sync(kt);
        pair_c(kt, B0{});
        tile_sync(kt + 1);
        pair_c(kt + 1, B1{});
    }
    if (kt < ntile) {
        tile_sync(kt);
        pair_c(kt, B0{});
    }

    if (kj < T) {
        store_row<D>(dk + goff, kj, half, dk_acc, scale, grs);
        store_row<D>(dv + goff, kj, half, dv_acc, 1.0f, grs);
    }
}

template <int D, int NSUB>
void dq_launch(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* o,
               const uint16_t* dO, const float* m, const float* l, uint16_t* dq, float* Dws,
               int BH, int T, float scale, const HeadView& xv, const HeadView& ov,
               const HeadView& gv, hipStream_t stream) {
    constexpr int kBlock = kWaves * NSUB * kSub;
    const int nblk = (T + kBlock - 1) / kBlock;
    hipLaunchKernelGGL((flash_bwd_dq_bf16_kernel<D, NSUB>), dim3(BH * nblk),
                       dim3(kWave * kWaves), 0, stream, q, k, v, o, dO, m, l, dq, Dws, BH, T,
                       scale, nblk, xv, ov, gv);
}

template <int D>
void dq_dispatch(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* o,
                 const uint16_t* dO, const float* m, const float* l, uint16_t* dq, float* Dws,
                 int BH, int T, float scale, const HeadView& xv, const HeadView& ov,
                 const HeadView& gv, hipStream_t stream) {
    // d = 128 holds one sub-block per wave (registers)
    if (D >= 128 || use_single_subblock(BH, T))
        dq_launch<D, 1>(q, k, v, o, dO, m, l, dq, Dws, BH, T, scale, xv, ov, gv, stream);
    else
        dq_launch<D, (D >= 128 ? 1 : 2)>(q, k, v, o, dO, m, l, dq, Dws, BH, T, scale, xv, ov, gv,
                                         stream);
}

template <int D>
void dkdv_dispatch(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* dO,
                   const float* m, const float* l, const float* Dws, uint16_t* dk, uint16_t* dv,
                   int BH, int T, float scale, const HeadView& xv, const HeadView& ov,
                   const HeadView& gv, hipStream_t stream) {
    constexpr int NW = kWaves;
    constexpr int kBlock = NW * kSub;
    const int nblk = (T + kBlock - 1) / kBlock;
    hipLaunchKernelGGL((flash_bwd_dkdv_bf16_kernel<D, NW>), dim3(BH * nblk), dim3(kWave * NW), 0,
                       stream, q, k, v, dO, m, l, Dws, dk, dv, BH, T, scale, nblk, xv, ov, gv);
}

}  // namespace

void launch_flash_bwd_dq_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                              const uint16_t* o, const uint16_t* dO, const float* m,
                              const float* l, uint16_t* dq, float* Dws, int BH, int T, int d,
                              float scale, const HeadView& xv, const HeadView& ov,
                              const HeadView& gv, hipStream_t stream) {
    switch (d) {
        case 32: dq_dispatch<32>(q, k, v, o, dO, m, l, dq, Dws, BH, T, scale, xv, ov, gv, stream); break;
        case 64: dq_dispatch<64>(q, k, v, o, dO, m, l, dq, Dws, BH, T, scale, xv, ov, gv, stream); break;
        default: dq_dispatch<128>(q, k, v, o, dO, m, l, dq, Dws, BH, T, scale, xv, ov, gv, stream); break;
    }
}

void launch_flash_bwd_dkdv_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                const uint16_t* dO, const float* m, const float* l,
                                const float* Dws, uint16_t* dk, uint16_t* dv, int BH, int T,
                                int d, float scale, const HeadView& xv, const HeadView& ov,
                                const HeadView& gv, hipStream_t stream) {
    switch (d) {
        case 32: dkdv_dispatch<32>(q, k, v, dO, m, l, Dws, dk, dv, BH, T, scale, xv, ov, gv, stream); break;
        case 64: dkdv_dispatch<64>(q, k, v, dO, m, l, Dws, dk, dv, BH, T, scale, xv, ov, gv, stream); break;
        default: dkdv_dispatch<128>(q, k, v, dO, m, l, Dws, dk, dv, BH, T, scale, xv, ov, gv, stream); break;
    }
}

}  // namespace tcamd
