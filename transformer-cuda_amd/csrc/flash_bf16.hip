// flash_bf16.hip - tiled causal attention backward on v_mfma_f32_32x32x16_bf16 with fp32
// accumulation (the forward is in flash_bf16_fwd.hip), for bf16 operands (NP = 1) and for
// fp32 operands carried as NP = 3 bf16 planes (bf16_tile.hpp).
//
// Algorithm: the reference's analytical backward (src/kernels/attention.cu:626-955) in the
// split form of the fp32 path: stage 1 (query-parallel) writes D = rowsum(dO * O) and dQ,
// stage 2 (key-parallel) dK and dV, both recomputing P = 2^(s*c - lse2) from the forward's
// statistics (lse2 = m*log2 e + log2 l, the log2-domain log-sum-exp).  P and dS are MFMA
// operands in NP planes (NP = 1: rounded to bf16); dQ/dK/dV are stored in bf16 (NP = 1,
// rounded once) or fp32 (NP = 3).
//
// Both stages use the forward's staging: tiles copied HBM -> LDS with
// global_load_lds_dwordx4 into XOR-swizzled rows, double buffered and shared by the 4 waves
// of a workgroup (NP planes per tile).  A product that contracts over the head dimension
// reads its A operand as 16-byte row reads of a tile and its B operand from VGPRs; a
// product that contracts over the sequence reads its A operand with ds_read_tr16_b64 from
// the same row-major tile and takes its B operand (P or dS) straight from the accumulator of
// the score product, whose rows are the contracted positions.  With NP = 3 the tiles come
// from plane tensors in HBM and the register operands are split from the fp32 rows.
//
// Stage 1, per 32-key half tile and 32-query sub-block (d = 64, NP = 1: 12 MFMAs):
//   S'^T = K (cQ)^T - lse2   A = K rows, B = c*Q (VGPRs), accumulator from -lse2
//   dP'^T = V dO^T - D       A = V rows, B = dO (VGPRs), accumulator from -D
//   dS^T = 2^S'^T o dP'^T    lane l holds query l%32
//   dQ^T += K^T dS^T         A = K^T (transposing reads of the K tile), B = dS^T
// Lane l's -lse2 and -D are the same in all 16 rows of its accumulators, so the products
// start from them (no statistic contraction step).  A workgroup owns 128 queries, one
// 32-query sub-block per wave.  NP = 3 streams 32-key tiles, so that the double-buffered K
// and V planes leave room for two workgroups per CU.
//
// Stage 2, per 32-query half tile and a wave's 32 keys (d = 64, NP = 1: 18 MFMAs):
//   S  = Q K^T        A = Q rows,  B = K (VGPRs)
//   dP = dO V^T       A = dO rows, B = V (VGPRs)
//   dS = P o (dP - D)              -lse2 and -D enter S and dP as one more contraction step
//                                  over a per-row statistic chunk held in LDS (see
//                                  dkdv_scores); K is held pre-multiplied by
//                                  c = scale*log2 e, so P = 2^S needs no per-element multiply
//   dV^T += dO^T P    A = dO^T (transposing reads), B = P
//   dK^T += Q^T dS    A = Q^T (transposing reads),  B = dS
// A workgroup owns 128 keys; query tiles start at the workgroup's first key, and wave w
// joins at the half tile that holds its first key (the only one it masks).  A wave handles
// both half tiles of a 64-query tile per step, so the MFMAs of one overlap the softmax
// arithmetic of the other.
//
// With NP = 3 the backward also runs in the dS-first order (its section below): D and the
// planes of dO first (bwd_prep_f32x3_kernel), then stage 2 writing dS in fp32 as well, then
// dQ = scale * dS K from the stored dS (flash_bwd_dq_ds_kernel), without stage 1's second
// computation of S and dP.
#include <math.h>

#include <type_traits>
#include <utility>

#include "bf16_tile.hpp"
#include "device_common.hpp"
#include "launch.hpp"
#include "sched.hpp"

namespace tcamd {
namespace {

using namespace bf16t;

// Element types: register-operand rows (bf16 or fp32) and outputs.
template <int NP>
using InT = std::conditional_t<NP == 1, uint16_t, float>;
template <int NP>
using OutT = std::conditional_t<NP == 1, uint16_t, float>;

// Key rows per stage-1 tile and query rows per stage-2 tile: NP = 3 streams 32-row tiles, so
// that the double-buffered planes leave room for two workgroups per CU.
template <int NP>
constexpr int kKeyTileDq = NP == 1 ? kRowTile : 32;
template <int NP>
constexpr int kQueryTile = NP == 1 ? kRowTile : 32;

// The three-plane dK/dV stage walks its query tiles from the last to the first.  dK and dV
// accumulate over every query in the MFMA accumulator (no register is left for compensated
// tile sums), and for a key the terms P_ij dO_i and dS_ij q_i shrink with the query index
// i (P_ij ~ 1/(i+1)): added small ones first, each is rounded against a smaller partial
// sum.
template <int NP>
constexpr bool kDesc = NP == 3;

// K and V tiles of stage 1 (as the forward's), NP planes each.  At d >= 64 the row stores of
// dO's planes and of dQ go through LDS stages inside an idle buffer.
template <int D, int NP>
struct KvSmem {
    uint16_t k[2][NP][Swz<D, kKeyTileDq<NP>>::kBytes / 2];
    uint16_t v[2][NP][Swz<D, kKeyTileDq<NP>>::kBytes / 2];
    static_assert(D < 64 || 2 * kStageBytes<D, NP> <= NP * Swz<D, kKeyTileDq<NP>>::kBytes,
                  "two wave stages per idle K (or V) buffer");
};

// Q and dO tiles of stage 2 (NP planes each), and per row an 8-element chunk that carries
// the row's statistic (see dkdv_scores).
template <int D, int NP>
struct QgSmem {
    static constexpr int KT = kQueryTile<NP>;
    uint16_t q[2][NP][Swz<D, KT>::kBytes / 2];
    uint16_t g[2][NP][Swz<D, KT>::kBytes / 2];
    uint16_t qx[2][KT * 8];  // row r: the terms of -lse2, then zeros
    uint16_t gx[2][KT * 8];  // row r: the terms of -D, then zeros
    // bf16 operands at d >= 64: the row stores of dK and dV go through LDS stages inside an
    // idle buffer (measured slower for the three-plane kernel, which stores directly)
    static_assert(NP != 1 || D < 64 || 2 * kStageBytes<D, NP> <= NP * Swz<D, KT>::kBytes,
                  "two wave stages per idle Q (or dO) buffer");
};

// A register operand over the head dimension: the NP planes of row `row` of a head (rows rs
// elements apart; zeros if row >= T), times `mul` first when SCALE (NP = 1: the bf16 value
// times mul, rounded to bf16 again; NP = 3: the fp32 value times mul, then split).
template <int D, int NP, bool SCALE>
__device__ __forceinline__ void load_operand(bf16x8 (&dst)[D / 16][NP],
                                             const InT<NP>* __restrict__ head, int row, int T,
                                             int half, int rs, float mul) {
    if constexpr (NP == 1) {
        bf16x8 t[D / 16];
        load_rowop<D>(t, head, row, T, half, rs);
#pragma unroll
        for (int st = 0; st < D / 16; ++st) {
            if constexpr (SCALE) {
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    t[st][e] = static_cast<__bf16>(static_cast<float>(t[st][e]) * mul);
            }
            dst[st][0] = t[st];
        }
    } else {
#pragma unroll
        for (int st = 0; st < D / 16; ++st) {
            float x[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            if (row < T) {
                const float* p = head + static_cast<size_t>(row) * rs + 16 * st + 8 * half;
                const f32x4 a = *reinterpret_cast<const f32x4*>(p);
                const f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    x[e] = SCALE ? a[e] * mul : a[e];
                    x[e + 4] = SCALE ? b[e] * mul : b[e];
                }
            }
            split_planes<NP>(x, dst[st]);
        }
    }
}

// ---------------------------------------------------------------------------------------
// Stage 1: D and dQ.
// ---------------------------------------------------------------------------------------

// The 32-query sub-block of a wave.  A lane holds one query, so its statistics are the same
// in all 16 rows of its accumulators: S^T and dP^T start from them (a 16-register copy of
// each per lane, kept for the whole task, exact in fp32), where one more contraction step
// (the A operand ones times a statistic chunk) would cost two MFMAs per half tile.
template <int D, int NP>
struct DqSub {
    bf16x8 q[D / 16][NP];  // c * Q row of query col (B operand over d)
    bf16x8 g[D / 16][NP];  // dO row
    f32x16 ls, ld;         // -lse2 (-1e30 for padded queries: P = 0) and -D in every row
    f32x16 acc[D / 32];    // dQ^T
};

// D = rowsum(dO o O) of an fp32 row, the share of lane half `half`: the dot products of the
// 8-element chunks 2j + half (an fma chain each, elements in order), summed as a pairwise
// tree over j; xhalf_sum of the two shares completes the row.  The same sums, in the same
// order, as bwd_prep_f32x3_kernel's butterfly over the chunks.
template <int D>
__device__ __forceinline__ float chunk_dot_tree(const float* __restrict__ gp,
                                                const float* __restrict__ op, int half) {
    float c[D / 16];
#pragma unroll
    for (int j = 0; j < D / 16; ++j) {
        c[j] = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e += 4) {
            const f32x4 a = *reinterpret_cast<const f32x4*>(gp + 16 * j + 8 * half + e);
            const f32x4 b = *reinterpret_cast<const f32x4*>(op + 16 * j + 8 * half + e);
#pragma unroll
            for (int i = 0; i < 4; ++i) c[j] = fmaf(a[i], b[i], c[j]);
        }
    }
#pragma unroll
    for (int w = 1; w < D / 16; w *= 2) {
#pragma unroll
        for (int j = 0; j < D / 16; j += 2 * w) c[j] += c[j + w];
    }
    return c[0];
}

// qh: this head's q (rows qrs apart); oh, gh: its o and dO (rows ors apart).  Q is held
// pre-multiplied by c = scale*log2 e (NP = 1: rounded to bf16, one extra rounding of ~2^-9
// relative per element; NP = 3: in fp32, then split), so that the scores come out in the
// log2 domain.  D = rowsum(dO o O) in fp32 from the stored O and dO.
template <int D, int NP>
__device__ __forceinline__ void dq_init(DqSub<D, NP>& sb, const InT<NP>* __restrict__ qh,
                                        const InT<NP>* __restrict__ oh,
                                        const InT<NP>* __restrict__ gh,
                                        const float* __restrict__ m, const float* __restrict__ l,
                                        float* __restrict__ Dws, int qrs, int ors,
                                        size_t stat_off, int qi, int T, int half, float c) {
    load_operand<D, NP, false>(sb.g, gh, qi, T, half, ors, 1.0f);
    float part = 0.0f;
    if constexpr (NP == 1) {
        bf16x8 orow[D / 16];
        load_rowop<D>(orow, oh, qi, T, half, ors);
#pragma unroll
        for (int j = 0; j < D / 16; ++j) {
#pragma unroll
            for (int e = 0; e < 8; ++e)
                part = fmaf(static_cast<float>(sb.g[j][0][e]), static_cast<float>(orow[j][e]),
                            part);
        }
    } else if (qi < T) {
        part = chunk_dot_tree<D>(gh + static_cast<size_t>(qi) * ors,
                                 oh + static_cast<size_t>(qi) * ors, half);
    }
    load_operand<D, NP, true>(sb.q, qh, qi, T, half, qrs, c);
    const float dlt = xhalf_sum(part);
    float nl = -1e30f;
    if (qi < T) {
        if (half == 0) Dws[stat_off + qi] = dlt;
        nl = -(m[stat_off + qi] * kLog2e + log2f(l[stat_off + qi]));
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        sb.ls[r] = nl;
        sb.ld[r] = -dlt;
    }
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) sb.acc[dt] = f32x16{};
}

// s = S'^T = K (cQ)^T - lse2, dp = dP'^T = V dO^T - D of keys kb.. (rows) x queries qj + col
// (columns) -> dS^T = 2^s o dp as the two B operands (NP planes each) of dQ^T += K^T dS^T.
// MASK: the half tile crosses the diagonal of the sub-block (keys past the query get P = 0);
// a compile-time flag, so that the other half tiles carry no compare and select per score.
template <int NP, bool MASK>
__device__ __forceinline__ void dq_ds(f32x16& s, const f32x16& dp, bf16x8 (&db)[2][NP], int kb,
                                      int qj, int col, int half) {
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = exp2_fast(s[r]);
    if constexpr (MASK) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
            if (kb + acc_row(r, half) > qj + col) s[r] = 0.0f;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] *= dp[r];
    pack_planes<NP>(s, 0, db[0]);
    pack_planes<NP>(s, 1, db[1]);
}

// One 32-key half tile of the wave's sub-block (MASK: its diagonal one).  ka/va: this lane's
// row-read addresses in plane 0 of the K / V tile; kta: transposing-read addresses in plane
// 0 of the K tile; plane i lies i tile sizes further.  S^T and dP^T start from -lse2 and -D.
template <int D, int NP, bool MASK>
__device__ __forceinline__ void dq_half(int kb, const uint32_t (&ka)[D / 16],
                                        const uint32_t (&va)[D / 16],
                                        const uint32_t (&kta)[D / 32], DqSub<D, NP>& sb, int qj,
                                        int col, int half) {
    constexpr uint32_t kPlane = Swz<D, kKeyTileDq<NP>>::kBytes;
    f32x16 s = sb.ls;
#pragma unroll
    for (int st = 0; st < D / 16; ++st) {
        bf16x8 a[NP];
#pragma unroll
        for (int i = 0; i < NP; ++i) a[i] = lds_b128(ka[st] + i * kPlane);
        s = mma_planes<NP>(a, sb.q[st], s);
    }
    f32x16 p = sb.ld;
#pragma unroll
    for (int st = 0; st < D / 16; ++st) {
        bf16x8 a[NP];
#pragma unroll
        for (int i = 0; i < NP; ++i) a[i] = lds_b128(va[st] + i * kPlane);
        p = mma_planes<NP>(a, sb.g[st], p);
    }
    bf16x8 d[2][NP];
    dq_ds<NP, MASK>(s, p, d, kb, qj, col, half);
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            bf16x8 a[NP];
#pragma unroll
            for (int i = 0; i < NP; ++i)
                a[i] = lds_tr(kta[dt] + i * kPlane + u * Swz<D>::rows(16), Swz<D>::rows(8));
            sb.acc[dt] = mma_planes<NP>(a, d[u], sb.acc[dt]);
        }
    }
}

// Operands of one stage-1 launch.  q, o, dO: register-operand rows (views qv, ov); k, v:
// plane 0 of the K / V tile sources (view kv, planes pstride elements apart); dq: output
// rows (view gv).
template <int NP>
struct DqArgs {
    const InT<NP> *q, *o, *dO;
    const uint16_t *k, *v;
    const float *m, *l;
    OutT<NP>* dq;
    float* Dws;
    int BH, T;
    float scale;
    HeadView qv, kv, ov, gv;
    size_t pstride;
    uint16_t* gp;  // dO planes out (NP = 3; laid out as k's), or null
    int serp;      // map_block's serpentine order (set at launch)
};

// 128 queries per workgroup, wave w owns the 32-query sub-block w.
template <int D, int NP>
__global__ __launch_bounds__(kWave* kWaves) void flash_bwd_dq_bf16_kernel(DqArgs<NP> a,
                                                                         int nblk) {
    constexpr int KT = kKeyTileDq<NP>;
    constexpr int kHalves = KT / 32;
    using S = Swz<D, KT>;
    constexpr uint32_t kBuf = NP * S::kBytes;  // one K (or V) buffer: NP plane tiles
    constexpr int kBlock = kWaves * kSub;
    __shared__ __attribute__((aligned(1024))) KvSmem<D, NP> sm;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int lane = threadIdx.x & (kWave - 1);
    const int col = lane & 31;
    const int half = lane >> 5;
    const int T = a.T;
    int bh, blk;
    map_block(blockIdx.x, a.BH, nblk, true, a.serp != 0, bh, blk);
    const int q0 = blk * kBlock;
    const int qj = q0 + kSub * wave;
    const size_t qoff = a.qv.off(bh), koff = a.kv.off(bh), ooff = a.ov.off(bh),
                 goff = a.gv.off(bh);
    const int krs = a.kv.row;
    const size_t stat_off = static_cast<size_t>(bh) * T;
    const uint16_t* kh = a.k + koff;
    const uint16_t* vh = a.v + koff;
    const float c = a.scale * kLog2e;

    const int kend = min(T, q0 + kBlock);
    const int ntile = (kend + KT - 1) / KT;
    const uint32_t k_lds = lds_addr(sm.k[0][0]);
    const uint32_t v_lds = lds_addr(sm.v[0][0]);
    // Tile kt of K and V (every plane) into buffer kt % 2.
    auto copy_tile = [&](int kt) {
        const uint32_t buf = static_cast<uint32_t>(kt & 1) * kBuf;
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            dma_tile<D, kWaves, KT>(kh + i * a.pstride, kt * KT, T, k_lds + buf + i * S::kBytes,
                                    wave, lane, krs);
            dma_tile<D, kWaves, KT>(vh + i * a.pstride, kt * KT, T, v_lds + buf + i * S::kBytes,
                                    wave, lane, krs);
        }
    };
    copy_tile(0);

    DqSub<D, NP> sb;
    dq_init<D, NP>(sb, a.q + qoff, a.o + ooff, a.dO + ooff, a.m, a.l, a.Dws, a.qv.row,
                   a.ov.row, stat_off, qj + col, T, half, c);
    if constexpr (NP > 1) {
        if (a.gp != nullptr) store_planes<D, NP>(a.gp + koff, a.pstride, sb.g, qj + col, T, half);
    }

    uint32_t roff[D / 16], troff[D / 32];
    lane_offsets<D>(lane, roff, troff);

    const int nhalf_t = (T + 31) / 32;
    const int hB = min(qj / 32 + 1, nhalf_t);  // half tiles of this wave; the last one masks
    const int hend = kHalves * ntile;
    uint32_t ka[D / 16], va[D / 16], kta[D / 32];
    auto tile_sync = [&](int hh) {
        const int kt = hh / kHalves;
        if (hh % kHalves == 0) {
            wait_vm<0>();     // this wave's copies of tile kt landed ...
            __syncthreads();  // ... and every wave's; tile kt-1 is no longer read by anyone
            if (kt + 1 < ntile) copy_tile(kt + 1);
        }
        const uint32_t base = static_cast<uint32_t>(kt & 1) * kBuf +
                              static_cast<uint32_t>(hh % kHalves) * S::rows(32);
#pragma unroll
        for (int st = 0; st < D / 16; ++st) {
            ka[st] = k_lds + base + roff[st];
            va[st] = v_lds + base + roff[st];
        }
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) kta[dt] = k_lds + base + troff[dt];
    };
    // the wave's half tiles 0 .. hB-2 unmasked, then its diagonal one (hB = 0: none)
    int hh = 0;
    for (; hh + 1 < hB; ++hh) {
        tile_sync(hh);
        dq_half<D, NP, false>(32 * hh, ka, va, kta, sb, qj, col, half);
    }
    if (hh < hB) {
        tile_sync(hh);
        dq_half<D, NP, true>(32 * hh, ka, va, kta, sb, qj, col, half);
        ++hh;
    }
    for (; hh < hend; ++hh) tile_sync(hh);

    if constexpr (D >= 64) {
        // after the last tile barrier the buffer without the last tile is idle
        const uint32_t stage = wave_stage(lds_addr(sm.k[ntile & 1][0]),
                                          lds_addr(sm.v[ntile & 1][0]), wave, kStageBytes<D, NP>);
        store_row_staged<D>(a.dq + goff, qj, T, lane, sb.acc, a.scale, a.gv.row, stage);
    } else {
        if (qj + col < T) store_row<D>(a.dq + goff, qj + col, half, sb.acc, a.scale, a.gv.row);
    }
}

// ---------------------------------------------------------------------------------------
// Stage 2: dK, dV.
// ---------------------------------------------------------------------------------------

// Per-lane operands of one 32-query half tile of stage 2 (plane 0; plane i lies i tile
// sizes further).
template <int D>
struct HalfAddr {
    uint32_t q[D / 16], g[D / 16];    // row reads, chunk step st
    uint32_t qt[D / 32], gt[D / 32];  // transposing reads, head-dim tile dt
    uint32_t qx, gx;                  // statistic chunks of row col
};

// S' = Q (cK)^T - lse2 and dP' = dO V^T - D of one half tile.  The statistics ride in the
// products: one more 16-wide contraction step multiplies the row's chunk (terms, 0, ...)
// by the B operand `one` = (1, 1, [1,] 0, ...) (lanes of k-group 1 hold zeros), so that
// 2^S' = P and P o dP' = dS need no per-row values in VGPRs.
template <int D, int NP>
__device__ __forceinline__ void dkdv_scores(const HalfAddr<D>& a, const bf16x8 (&kr)[D / 16][NP],
                                            const bf16x8 (&vr)[D / 16][NP], const bf16x8& one,
                                            f32x16& s, f32x16& dp) {
    constexpr uint32_t kPlane = Swz<D, kQueryTile<NP>>::kBytes;
    s = mfma_32x32x16_bf16(lds_b128(a.qx), one, f32x16{});
#pragma unroll
    for (int st = 0; st < D / 16; ++st) {
        bf16x8 x[NP];
#pragma unroll
        for (int i = 0; i < NP; ++i) x[i] = lds_b128(a.q[st] + i * kPlane);
        s = mma_planes<NP>(x, kr[st], s);
    }
    dp = mfma_32x32x16_bf16(lds_b128(a.gx), one, f32x16{});
#pragma unroll
    for (int st = 0; st < D / 16; ++st) {
        bf16x8 x[NP];
#pragma unroll
        for (int i = 0; i < NP; ++i) x[i] = lds_b128(a.g[st] + i * kPlane);
        dp = mma_planes<NP>(x, vr[st], dp);
    }
}

// Where a wave's dS values of a 32-query step go: the step's dS tile (wave-uniform; rows
// ld = 32 elements apart); the lane's element of accumulator row r is at
// row + (8*(r/4) + r%4)*ld + lane_off (lane_off = 4*half*ld + the key's column in the tile).
// zero: the lane's key lies past T (written as zeros).
struct DsOut {
    float* row = nullptr;
    int ld = 0;
    uint32_t lane_off = 0;
    bool zero = false;
};

// P = 2^S' (0 where the query precedes the key, on the diagonal half tile) and
// dS = P o dP'; dV^T += dO^T P, dK^T += Q^T dS.
template <int D, bool MASK, int NP, bool DS = false>
__device__ __forceinline__ void dkdv_update(const HalfAddr<D>& a, f32x16& s, const f32x16& dp,
                                            f32x16 (&dk_acc)[D / 32],
                                            f32x16 (&dv_acc)[D / 32], int qb, int kj,
                                            int half, const DsOut& dso = DsOut{}) {
    constexpr uint32_t kPlane = Swz<D, kQueryTile<NP>>::kBytes;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = exp2_fast(s[r]);
    if constexpr (MASK) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
            if (qb + acc_row(r, half) < kj) s[r] = 0.0f;
    }
    if constexpr (NP == 1) {
        bf16x8 pb[2][NP], db[2][NP];
        pack_planes<NP>(s, 0, pb[0]);
        pack_planes<NP>(s, 1, pb[1]);
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] *= dp[r];
        pack_planes<NP>(s, 0, db[0]);
        pack_planes<NP>(s, 1, db[1]);
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                bf16x8 g[NP], q[NP];
#pragma unroll
                for (int i = 0; i < NP; ++i) {
                    g[i] = lds_tr(a.gt[dt] + i * kPlane + u * Swz<D>::rows(16), Swz<D>::rows(8));
                    q[i] = lds_tr(a.qt[dt] + i * kPlane + u * Swz<D>::rows(16), Swz<D>::rows(8));
                }
                dv_acc[dt] = mma_planes<NP>(g, pb[u], dv_acc[dt]);
                dk_acc[dt] = mma_planes<NP>(q, db[u], dk_acc[dt]);
            }
        }
    } else {
        // Planes of P, then of dS, one 16-row half at a time: fewer live registers.
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            bf16x8 pb[NP];
            pack_planes<NP>(s, u, pb);
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt) {
                bf16x8 g[NP];
#pragma unroll
                for (int i = 0; i < NP; ++i)
                    g[i] = lds_tr(a.gt[dt] + i * kPlane + u * Swz<D>::rows(16), Swz<D>::rows(8));
                dv_acc[dt] = mma_planes<NP>(g, pb, dv_acc[dt]);
            }
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] *= dp[r];
        // a 32-lane store covers one query's 32 keys (128 bytes); nontemporal, so that dS
        // (read once, by the next kernel) does not push the Q/dO plane tiles out of L2 (config
        // 2 step 346.7 -> 343.1 us; the fp32 kernel's plain stores measured faster there)
        if constexpr (DS) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                float* row = dso.row + static_cast<size_t>(8 * (r / 4) + r % 4) * dso.ld;
                __builtin_nontemporal_store(dso.zero ? 0.0f : s[r], row + dso.lane_off);
            }
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            bf16x8 db[NP];
            pack_planes<NP>(s, u, db);
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt) {
                bf16x8 q[NP];
#pragma unroll
                for (int i = 0; i < NP; ++i)
                    q[i] = lds_tr(a.qt[dt] + i * kPlane + u * Swz<D>::rows(16), Swz<D>::rows(8));
                dk_acc[dt] = mma_planes<NP>(q, db, dk_acc[dt]);
            }
        }
    }
}

// Operands of one stage-2 launch.  q, dO: plane 0 of the Q / dO tile sources (views qv,
// gtv; planes pstride elements apart); k, v: register-operand rows (view kv); dk, dv:
// output rows (view gv).
template <int NP>
struct DkdvArgs {
    const uint16_t *q, *dO;
    const InT<NP> *k, *v;
    const float *m, *l, *Dws;
    OutT<NP> *dk, *dv;
    int BH, T;
    float scale;
    HeadView qv, gtv, kv, gv;
    size_t pstride;
    // NP = 3, optional: dS out (fp32), for a dQ stage that reads it instead of recomputing S
    // and dP: the 32 x 32 tiles of ds_tile (ds_n = T rounded up to 32) at or below the
    // diagonal, keys >= T as zeros.
    float* ds = nullptr;
    int ds_n = 0;
    int group = 0;  // heads per group of map_block_grouped (NP = 1; set at launch), 0: none
};

// NW waves per workgroup; wave w owns keys k0 + 32w ...  DS: write dS out (NP = 3, a.ds).
template <int D, int NW, int NP, bool DS = false>
__global__ __launch_bounds__(kWave* NW, NP == 1 ? 1 : 2) void flash_bwd_dkdv_bf16_kernel(DkdvArgs<NP> a,
                                                                       int nblk) {
    constexpr int KT = kQueryTile<NP>;
    using S = Swz<D, KT>;
    constexpr uint32_t kBuf = NP * S::kBytes;  // one Q (or dO) buffer: NP plane tiles
    constexpr int kBlock = NW * kSub;          // keys per workgroup
    __shared__ __attribute__((aligned(1024))) QgSmem<D, NP> sm;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int lane = threadIdx.x & (kWave - 1);
    const int col = lane & 31;
    const int half = lane >> 5;
    const int T = a.T;
    int bh, blk;
    map_block(blockIdx.x, a.BH, nblk, false, false, bh, blk);  // block 0 sees every query
    const int k0 = blk * kBlock;
    const int kw = k0 + kSub * wave;
    const int kj = kw + col;
    const size_t qoff = a.qv.off(bh), gtoff = a.gtv.off(bh), koff = a.kv.off(bh),
                 goff = a.gv.off(bh);
    const int qrs = a.qv.row, grs = a.gtv.row;
    const size_t stat_off = static_cast<size_t>(bh) * T;
    const uint16_t* qh = a.q + qoff;
    const uint16_t* gh = a.dO + gtoff;
    const float c = a.scale * kLog2e;

    const int t0 = k0 / KT;
    const int ntile = (T + KT - 1) / KT;
    // Three planes walk the query tiles downward (kDesc): the last tile first, the
    // workgroup's first key's tile last.
    const int tfirst = kDesc<NP> ? ntile - 1 : t0;
    const uint32_t q_lds = lds_addr(sm.q[0][0]);
    const uint32_t g_lds = lds_addr(sm.g[0][0]);
    const uint32_t qx_lds = lds_addr(sm.qx[0]);
    const uint32_t gx_lds = lds_addr(sm.gx[0]);
    // Tile kt of Q and dO (every plane) into buffer kt % 2.
    auto copy_tile = [&](int kt) {
        const uint32_t buf = static_cast<uint32_t>(kt & 1) * kBuf;
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            dma_tile<D, NW, KT>(qh + i * a.pstride, kt * KT, T, q_lds + buf + i * S::kBytes,
                                wave, lane, qrs);
            dma_tile<D, NW, KT>(gh + i * a.pstride, kt * KT, T, g_lds + buf + i * S::kBytes,
                                wave, lane, grs);
        }
    };
    copy_tile(tfirst);
    // Wave 0 stages the statistics of a tile through VGPRs: lane i < KT holds query KT*t + i.
    float st_m = 0.0f, st_l = 1.0f, st_d = 0.0f;
    auto load_stats = [&](int t) {
        const int r = t * KT + lane;
        if (r < T) {
            st_m = a.m[stat_off + r];
            st_l = a.l[stat_off + r];
            st_d = a.Dws[stat_off + r];
        } else {
            st_m = -INFINITY;  // padded query: P = 0 (see tile_sync)
            st_l = 1.0f;
            st_d = 0.0f;
        }
    };
    if (wave == 0 && lane < KT) {
        load_stats(tfirst);
        const u16x8 z = u16x8{};  // the constant zeros of the statistic chunks
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            *reinterpret_cast<u16x8*>(&sm.qx[b][lane * 8]) = z;
            *reinterpret_cast<u16x8*>(&sm.gx[b][lane * 8]) = z;
        }
    }
    const bf16x8 one = ones_chunk<NP>(half);

    // c*K (NP = 1: rounded to bf16, one extra rounding of ~2^-9 relative per element; the
    // score error it causes is a random sum over d, ~1e-3 in log2 units for unit-variance
    // inputs.  NP = 3: in fp32, then split) and V.
    bf16x8 kr[D / 16][NP], vr[D / 16][NP];
    load_operand<D, NP, true>(kr, a.k + koff, kj, T, half, a.kv.row, c);
    load_operand<D, NP, false>(vr, a.v + koff, kj, T, half, a.kv.row, 1.0f);
    f32x16 dk_acc[D / 32], dv_acc[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
        dk_acc[dt] = f32x16{};
        dv_acc[dt] = f32x16{};
    }
    uint32_t roff[D / 16], troff[D / 32];
    lane_offsets<D>(lane, roff, troff);
    const uint32_t soff = static_cast<uint32_t>(col * 16);  // statistic chunk of row col

    // Tile kt: wait for its copies, publish its statistics, barrier, start the next copy
    // (tile kt - 1 when descending).
    auto tile_sync = [&](int kt) {
        wait_vm<0>();  // this wave's copies (and statistics loads) of tile kt landed
        if (wave == 0 && lane < KT) {  // terms of -lse2 (-1e30 for padded queries: P = 0), -D
            const float nl = st_m == -INFINITY ? -1e30f : -(st_m * kLog2e + log2f(st_l));
            *reinterpret_cast<u16x4*>(&sm.qx[kt & 1][lane * 8]) = stat_terms<NP>(nl);
            *reinterpret_cast<u16x4*>(&sm.gx[kt & 1][lane * 8]) = stat_terms<NP>(-st_d);
        }
        __syncthreads();  // every wave's copies landed; the previous tile is no longer read
        const int nt = kDesc<NP> ? kt - 1 : kt + 1;
        if (kDesc<NP> ? nt >= t0 : nt < ntile) {
            if (wave == 0 && lane < KT) load_stats(nt);
            copy_tile(nt);
        }
    };
    // Operand addresses of half tile hh (queries 32*hh ..).
    auto half_addr = [&](int hh) {
        HalfAddr<D> h;
        const int kt = hh >> 1;
        const uint32_t base = static_cast<uint32_t>(kt & 1) * kBuf +
                              static_cast<uint32_t>(hh & 1) * S::rows(32);
#pragma unroll
        for (int st = 0; st < D / 16; ++st) {
            h.q[st] = q_lds + base + roff[st];
            h.g[st] = g_lds + base + roff[st];
        }
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) {
            h.qt[dt] = q_lds + base + troff[dt];
            h.gt[dt] = g_lds + base + troff[dt];
        }
        const uint32_t xrow = static_cast<uint32_t>(((kt & 1) * KT + (hh & 1) * 32 + col) * 16);
        h.qx = qx_lds + xrow;
        h.gx = gx_lds + xrow;
        return h;
    };
    // The same with the buffer parity and half a compile-time constant: every address is a
    // lane offset plus an immediate.
    auto half_addr_c = [&](auto buf, auto hsel) {
        HalfAddr<D> h;
        constexpr uint32_t base = static_cast<uint32_t>(decltype(buf)::value) * kBuf +
                                  static_cast<uint32_t>(decltype(hsel)::value) * S::rows(32);
        constexpr uint32_t xbase = static_cast<uint32_t>(decltype(buf)::value * KT +
                                                         decltype(hsel)::value * 32) * 16u;
#pragma unroll
        for (int st = 0; st < D / 16; ++st) {
            h.q[st] = roff[st] + (q_lds + base);
            h.g[st] = roff[st] + (g_lds + base);
        }
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) {
            h.qt[dt] = troff[dt] + (q_lds + base);
            h.gt[dt] = troff[dt] + (g_lds + base);
        }
        h.qx = soff + (qx_lds + xbase);
        h.gx = soff + (gx_lds + xbase);
        return h;
    };
    // Both half tiles of tile kt (held in buffer `buf`), no diagonal.
    auto pair_c = [&](int kt, auto buf) {
        const HalfAddr<D> a0 = half_addr_c(buf, std::integral_constant<int, 0>{});
        const HalfAddr<D> a1 = half_addr_c(buf, std::integral_constant<int, 1>{});
        f32x16 s0, dp0, s1, dp1;
        dkdv_scores<D, NP>(a0, kr, vr, one, s0, dp0);
        dkdv_scores<D, NP>(a1, kr, vr, one, s1, dp1);
        dkdv_update<D, false, NP>(a0, s0, dp0, dk_acc, dv_acc, 64 * kt, kj, half);
        dkdv_update<D, false, NP>(a1, s1, dp1, dk_acc, dv_acc, 64 * kt + 32, kj, half);
    };
    // Both half tiles of tile kt; the first is the diagonal one when MASK0.  The score
    // products of the second half tile are issued before the first half tile's softmax.
    auto pair = [&](int kt, auto mask0) {
        const HalfAddr<D> a0 = half_addr(2 * kt), a1 = half_addr(2 * kt + 1);
        f32x16 s0, dp0, s1, dp1;
        dkdv_scores<D, NP>(a0, kr, vr, one, s0, dp0);
        dkdv_scores<D, NP>(a1, kr, vr, one, s1, dp1);
        dkdv_update<D, decltype(mask0)::value, NP>(a0, s0, dp0, dk_acc, dv_acc, 64 * kt, kj,
                                                   half);
        dkdv_update<D, false, NP>(a1, s1, dp1, dk_acc, dv_acc, 64 * kt + 32, kj, half);
    };

    if constexpr (KT == 32) {
        // One 32-query tile per step.  Tiles before tstart (= kw/32, the one holding the
        // wave's first key, the only one it masks) hold only queries that precede every key
        // of the wave; a wave whose keys start past T computes nothing.  Every wave takes
        // part in every tile's barrier and copies.
        auto step = [&](int kt, auto mask) {
            HalfAddr<D> h;
            const uint32_t base = static_cast<uint32_t>(kt & 1) * kBuf;
#pragma unroll
            for (int st = 0; st < D / 16; ++st) {
                h.q[st] = q_lds + base + roff[st];
                h.g[st] = g_lds + base + roff[st];
            }
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt) {
                h.qt[dt] = q_lds + base + troff[dt];
                h.gt[dt] = g_lds + base + troff[dt];
            }
            const uint32_t xrow = static_cast<uint32_t>(((kt & 1) * KT + col) * 16);
            h.qx = qx_lds + xrow;
            h.gx = gx_lds + xrow;
            f32x16 s1, dp1;
            dkdv_scores<D, NP>(h, kr, vr, one, s1, dp1);
            DsOut dso;
            if constexpr (DS) {
                static_assert(!DS || KT == 32, "dS tiles are 32 queries deep");
                dso.row = a.ds + ds_tile(bh, a.ds_n, kt, kw / 32);
                dso.ld = 32;
                dso.lane_off = static_cast<uint32_t>(4 * half * 32 + col);
                dso.zero = kj >= T;
            }
            dkdv_update<D, decltype(mask)::value, NP, DS>(h, s1, dp1, dk_acc, dv_acc, KT * kt,
                                                          kj, half, dso);
        };
        const int tstart = kw < T ? kw / KT : ntile;
        if constexpr (kDesc<NP>) {
            // Downward: the wave's unmasked tiles, its diagonal tile, then barriers only.
            int kt = ntile - 1;
            for (; kt > tstart; --kt) {
                tile_sync(kt);
                step(kt, std::false_type{});
            }
            if (kt == tstart && kt < ntile) {
                tile_sync(kt);
                step(kt, std::true_type{});
                --kt;
            }
            for (; kt >= t0; --kt) tile_sync(kt);
        } else {
            int kt = t0;
            for (; kt < tstart; ++kt) tile_sync(kt);
            if (kt < ntile) {
                tile_sync(kt);
                step(kt, std::true_type{});
                ++kt;
            }
            for (; kt < ntile; ++kt) {
                tile_sync(kt);
                step(kt, std::false_type{});
            }
        }
    } else {
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
                dkdv_scores<D, NP>(a1, kr, vr, one, s1, dp1);
                dkdv_update<D, true, NP>(a1, s1, dp1, dk_acc, dv_acc, 32 * hstart, kj, half);
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

    }

    if (kj < T) {
        store_row<D>(a.dk + goff, kj, half, dk_acc, a.scale, a.gv.row);
        store_row<D>(a.dv + goff, kj, half, dv_acc, 1.0f, a.gv.row);
    }
}

// ---------------------------------------------------------------------------------------
// Stage 2 for bf16 operands with an explicit instruction schedule.
//
// The same products, in the same order per accumulator, as flash_bwd_dkdv_bf16_kernel<D, 4,
// 1> (so the same results, bit for bit), but issued as a fixed program per 64-query tile in
// which
//   * every MFMA's A fragment is read from LDS kRing - 1 MFMAs ahead, into a ring of kRing
//     fragments, so that an LDS read's latency is covered by the MFMAs before its
//     consumer (left to itself, the compiler reads each fragment into one reused register
//     quad just before its MFMA and waits for it: one exposed LDS latency per MFMA);
//   * the softmax arithmetic of a half tile is spread between the MFMAs of the next part of
//     the program: that of half 0 (2^S, mask, P, dS = P o dP', both packed to bf16) between
//     the score products of half 1, that of half 1 between the dV/dK products of half 0.
// The program of one wave and tile (NS = D/16 chunks over d, NDT = D/32 head-dim tiles):
//   ops [0, 2(NS+1))            half 0: S' (statistic step, NS chunks), dP' (the same)
//   ops [2(NS+1), 4(NS+1))      half 1: the same          + softmax arithmetic of half 0
//   ops [.., + 4 NDT)           half 0: for dt, u: dV, dK + softmax arithmetic of half 1
//   ops [.., + 4 NDT)           half 1: for dt, u: dV, dK
// sched_barrier fences around each op keep the compiler's scheduler from moving the
// program's instructions across ops.
// ---------------------------------------------------------------------------------------

template <int... Is, typename F>
__device__ __forceinline__ void static_for_impl(std::integer_sequence<int, Is...>, F&& f) {
    (f(std::integral_constant<int, Is>{}), ...);
}
// f(integral_constant<int, 0>) ... f(integral_constant<int, N-1>), in order.
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(std::make_integer_sequence<int, N>{}, f);
}

__device__ __forceinline__ void sched_fence() { __builtin_amdgcn_sched_barrier(0); }

template <int D>
struct DkdvProgram {
    static constexpr int NS = D / 16;           // chunks of a score product
    static constexpr int NDT = D / 32;          // head-dim tiles of dV / dK
    static constexpr int kScores = 2 * (NS + 1);  // ops of one half's S' and dP'
    static constexpr int kUpd = 4 * NDT;          // ops of one half's dV and dK
    static constexpr int N = 2 * kScores + 2 * kUpd;
    static constexpr bool is_score(int i) { return i < 2 * kScores; }
    static constexpr int half(int i) {
        return i < 2 * kScores ? i / kScores : (i - 2 * kScores) / kUpd;
    }
    static constexpr int local(int i) {
        return i < 2 * kScores ? i % kScores : (i - 2 * kScores) % kUpd;
    }
    // A half's score ops alternate between its two products, S' (even local index) and dP'
    // (odd), so that consecutive MFMAs are independent (a lone dependent chain issues at
    // about 3/4 of the MFMA rate with one wave per SIMD); step 0 of each is the statistic
    // fold, steps 1..NS its head-dimension chunks.
    static constexpr bool score_dp(int j) { return j % 2 == 1; }
    static constexpr int score_step(int j) { return j / 2; }
    // Softmax task t (0..15) of a half runs at slot `slot(t, n)` of the n ops it overlaps:
    // tasks 0..7 take 2^S, mask and pack P for elements 2t, 2t+1; tasks 8..15 form and pack
    // dS for elements 2(t-8), 2(t-8)+1.
    static constexpr int slot(int t, int n) { return t * n / 16; }
};

// A fragments in flight: op i's fragment is read kRing - 1 ops ahead of its MFMA.
template <int D>
constexpr int kRing = D >= 128 ? 3 : 4;

// Per-wave state of one tile's program.
template <int D>
struct DkdvTileRegs {
    f32x16 s[2], dp[2];   // S' then P (in place), dP' per half
    bf16x8 p[2][2];       // P of half h, rows 16u.. (B operand of dV)
    bf16x8 ds[2][2];      // dS of half h (B operand of dK)
    bf16x8 ring[kRing<D>];
};

template <int D>
__global__ __launch_bounds__(kWave * kWaves, D >= 128 ? 1 : 2) void flash_bwd_dkdv_bf16_pipe_kernel(
    DkdvArgs<1> a, int nblk) {
    using Prog = DkdvProgram<D>;
    constexpr int KT = kRowTile;
    using S = Swz<D, KT>;
    constexpr uint32_t kBuf = S::kBytes;  // one Q (or dO) buffer
    constexpr int kBlock = kWaves * kSub;
    __shared__ __attribute__((aligned(1024))) QgSmem<D, 1> sm;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & (kWave - 1);
    const int col = lane & 31;
    const int half = lane >> 5;
    const int T = a.T;
    int bh, blk;
    map_block_grouped(blockIdx.x, a.BH, nblk, a.group, false, bh, blk);
    const int k0 = blk * kBlock;
    const int kw = k0 + kSub * wave;
    const int kj = kw + col;
    const size_t qoff = a.qv.off(bh), gtoff = a.gtv.off(bh), koff = a.kv.off(bh),
                 goff = a.gv.off(bh);
    const int qrs = a.qv.row, grs = a.gtv.row;
    const size_t stat_off = static_cast<size_t>(bh) * T;
    const uint16_t* qh = a.q + qoff;
    const uint16_t* gh = a.dO + gtoff;
    const float c = a.scale * kLog2e;

    const int t0 = k0 / KT;
    const int ntile = (T + KT - 1) / KT;
    const uint32_t q_lds = lds_addr(sm.q[0][0]);
    const uint32_t g_lds = lds_addr(sm.g[0][0]);
    const uint32_t qx_lds = lds_addr(sm.qx[0]);
    const uint32_t gx_lds = lds_addr(sm.gx[0]);
    auto copy_tile = [&](int kt) {
        const uint32_t buf = static_cast<uint32_t>(kt & 1) * kBuf;
        dma_tile<D, kWaves, KT>(qh, kt * KT, T, q_lds + buf, wave, lane, qrs);
        dma_tile<D, kWaves, KT>(gh, kt * KT, T, g_lds + buf, wave, lane, grs);
    };
    copy_tile(t0);
    float st_m = 0.0f, st_l = 1.0f, st_d = 0.0f;
    auto load_stats = [&](int t) {
        const int r = t * KT + lane;
        if (r < T) {
            st_m = a.m[stat_off + r];
            st_l = a.l[stat_off + r];
            st_d = a.Dws[stat_off + r];
        } else {
            st_m = -INFINITY;
            st_l = 1.0f;
            st_d = 0.0f;
        }
    };
    if (wave == 0 && lane < KT) {
        load_stats(t0);
        const u16x8 z = u16x8{};
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            *reinterpret_cast<u16x8*>(&sm.qx[b][lane * 8]) = z;
            *reinterpret_cast<u16x8*>(&sm.gx[b][lane * 8]) = z;
        }
    }
    const bf16x8 one = ones_chunk<1>(half);
    bf16x8 kr[D / 16][1], vr[D / 16][1];
    load_operand<D, 1, true>(kr, a.k + koff, kj, T, half, a.kv.row, c);
    load_operand<D, 1, false>(vr, a.v + koff, kj, T, half, a.kv.row, 1.0f);
    f32x16 dk_acc[D / 32], dv_acc[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
        dk_acc[dt] = f32x16{};
        dv_acc[dt] = f32x16{};
    }
    uint32_t roff[D / 16], troff[D / 32];
    lane_offsets<D>(lane, roff, troff);
    const uint32_t soff = static_cast<uint32_t>(col * 16);

    auto tile_sync = [&](int kt) {
        wait_vm<0>();
        if (wave == 0 && lane < KT) {
            const float nl = st_m == -INFINITY ? -1e30f : -(st_m * kLog2e + log2f(st_l));
            *reinterpret_cast<u16x4*>(&sm.qx[kt & 1][lane * 8]) = stat_terms<1>(nl);
            *reinterpret_cast<u16x4*>(&sm.gx[kt & 1][lane * 8]) = stat_terms<1>(-st_d);
        }
        __syncthreads();
        if (kt + 1 < ntile) {
            if (wave == 0 && lane < KT) load_stats(kt + 1);
            copy_tile(kt + 1);
        }
    };

    // A fragment of op I of the program (tile in buffer BUF).
    auto fetch = [&](auto buf, auto I) -> bf16x8 {
        constexpr int BUF = decltype(buf)::value;
        constexpr int i = decltype(I)::value;
        constexpr int h = Prog::half(i), j = Prog::local(i);
        constexpr uint32_t hb = static_cast<uint32_t>(BUF) * kBuf + static_cast<uint32_t>(h) * S::rows(32);
        constexpr uint32_t xb = static_cast<uint32_t>(BUF * KT + h * 32) * 16u;
        if constexpr (Prog::is_score(i)) {
            constexpr int st = Prog::score_step(j);
            if constexpr (!Prog::score_dp(j)) {
                if constexpr (st == 0) return lds_b128(soff + (qx_lds + xb));
                else return lds_b128(roff[st - 1] + (q_lds + hb));
            } else {
                if constexpr (st == 0) return lds_b128(soff + (gx_lds + xb));
                else return lds_b128(roff[st - 1] + (g_lds + hb));
            }
        } else {
            constexpr int p = j / 2, dt = p / 2, u = p % 2;
            constexpr uint32_t off = hb + static_cast<uint32_t>(u) * Swz<D>::rows(16);
            if constexpr (j % 2 == 0) return lds_tr(troff[dt] + (g_lds + off), Swz<D>::rows(8));
            else return lds_tr(troff[dt] + (q_lds + off), Swz<D>::rows(8));
        }
    };
    // The MFMA of op I with its A fragment x.
    auto product = [&](DkdvTileRegs<D>& r, auto I, const bf16x8& x) {
        constexpr int i = decltype(I)::value;
        constexpr int h = Prog::half(i), j = Prog::local(i);
        if constexpr (Prog::is_score(i)) {
            constexpr int st = Prog::score_step(j);
            if constexpr (!Prog::score_dp(j)) {
                if constexpr (st == 0) r.s[h] = mfma_32x32x16_bf16(x, one, f32x16{});
                else r.s[h] = mfma_32x32x16_bf16(x, kr[st - 1][0], r.s[h]);
            } else {
                if constexpr (st == 0) r.dp[h] = mfma_32x32x16_bf16(x, one, f32x16{});
                else r.dp[h] = mfma_32x32x16_bf16(x, vr[st - 1][0], r.dp[h]);
            }
        } else {
            constexpr int p = j / 2, dt = p / 2, u = p % 2;
            if constexpr (j % 2 == 0) dv_acc[dt] = mfma_32x32x16_bf16(x, r.p[h][u], dv_acc[dt]);
            else dk_acc[dt] = mfma_32x32x16_bf16(x, r.ds[h][u], dk_acc[dt]);
        }
    };
    // Softmax task T of half H (see DkdvProgram::slot); MASK: the half tile holds queries
    // before this lane's key (queries qb..qb+31).
    auto task = [&](DkdvTileRegs<D>& r, auto H, auto Tk, auto mask, int qb) {
        constexpr int h = decltype(H)::value, t = decltype(Tk)::value;
        constexpr int e = 2 * (t % 8), u = e / 8, k = e % 8;
        if constexpr (t < 8) {
            r.s[h][e] = exp2_fast(r.s[h][e]);
            r.s[h][e + 1] = exp2_fast(r.s[h][e + 1]);
            if constexpr (decltype(mask)::value) {
                if (qb + acc_row(e, half) < kj) r.s[h][e] = 0.0f;
                if (qb + acc_row(e + 1, half) < kj) r.s[h][e + 1] = 0.0f;
            }
            r.p[h][u][k] = static_cast<__bf16>(r.s[h][e]);
            r.p[h][u][k + 1] = static_cast<__bf16>(r.s[h][e + 1]);
        } else {
            r.ds[h][u][k] = static_cast<__bf16>(r.s[h][e] * r.dp[h][e]);
            r.ds[h][u][k + 1] = static_cast<__bf16>(r.s[h][e + 1] * r.dp[h][e + 1]);
        }
    };
    // The softmax tasks of half H that run at position k of a stretch of n ops.
    auto tasks_at = [&](DkdvTileRegs<D>& r, auto H, auto mask, int qb, auto K, auto Nn) {
        constexpr int kk = decltype(K)::value, n = decltype(Nn)::value;
        static_for<16>([&](auto Tk) {
            if constexpr (Prog::slot(decltype(Tk)::value, n) == kk) task(r, H, Tk, mask, qb);
        });
    };

    // Both half tiles of tile kt (buffer BUF); half 0 is the diagonal one when MASK0.
    auto full_tile = [&](int kt, auto buf, auto mask0) {
        constexpr int R = kRing<D>;
        DkdvTileRegs<D> r;
        static_for<R - 1>([&](auto I) { r.ring[decltype(I)::value] = fetch(buf, I); });
        const int qb = KT * kt;
        static_for<Prog::N>([&](auto I) {
            constexpr int i = decltype(I)::value;
            if constexpr (i + R - 1 < Prog::N)
                r.ring[(i + R - 1) % R] = fetch(buf, std::integral_constant<int, i + R - 1>{});
            sched_fence();
            product(r, I, r.ring[i % R]);
            if constexpr (i >= Prog::kScores && i < 2 * Prog::kScores)
                tasks_at(r, std::integral_constant<int, 0>{}, mask0, qb,
                         std::integral_constant<int, i - Prog::kScores>{},
                         std::integral_constant<int, Prog::kScores>{});
            if constexpr (i >= 2 * Prog::kScores && i < 2 * Prog::kScores + Prog::kUpd)
                tasks_at(r, std::integral_constant<int, 1>{}, std::false_type{}, qb + 32,
                         std::integral_constant<int, i - 2 * Prog::kScores>{},
                         std::integral_constant<int, Prog::kUpd>{});
            sched_fence();
        });
    };
    // Only half tile 1 of tile kt (buffer BUF), the diagonal one: no overlap.
    auto second_half_only = [&](int kt, auto buf) {
        DkdvTileRegs<D> r;
        constexpr int b = Prog::kScores;  // first op of half 1's scores
        constexpr int e = 2 * Prog::kScores + Prog::kUpd;  // first op of half 1's updates
        static_for<Prog::kScores>([&](auto I) {
            constexpr int i = b + decltype(I)::value;
            product(r, std::integral_constant<int, i>{}, fetch(buf, std::integral_constant<int, i>{}));
        });
        static_for<16>([&](auto Tk) {
            task(r, std::integral_constant<int, 1>{}, Tk, std::true_type{}, KT * kt + 32);
        });
        static_for<Prog::kUpd>([&](auto I) {
            constexpr int i = e + decltype(I)::value;
            product(r, std::integral_constant<int, i>{}, fetch(buf, std::integral_constant<int, i>{}));
        });
    };
    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;
    auto run_tile = [&](int kt, auto mask0) {
        if (kt & 1)
            full_tile(kt, B1{}, mask0);
        else
            full_tile(kt, B0{}, mask0);
    };

    // Half tiles before hstart (= kw/32, the one holding the wave's first key) hold only
    // queries that precede every key of the wave; a wave whose keys start past T computes
    // nothing.  Every wave takes part in every tile's barrier and copies.
    const int hstart = kw < T ? kw / 32 : 2 * ntile;
    int kt = t0;
    for (; 2 * kt + 1 < hstart; ++kt) tile_sync(kt);
    if (kt < ntile) {  // the tile holding the diagonal half tile
        tile_sync(kt);
        if (hstart & 1) {
            if (kt & 1)
                second_half_only(kt, B1{});
            else
                second_half_only(kt, B0{});
        } else {
            run_tile(kt, std::true_type{});
        }
        ++kt;
    }
    if (kt < ntile && (kt & 1)) {
        tile_sync(kt);
        full_tile(kt, B1{}, std::false_type{});
        ++kt;
    }
    for (; kt + 1 < ntile; kt += 2) {
        tile_sync(kt);
        full_tile(kt, B0{}, std::false_type{});
        tile_sync(kt + 1);
        full_tile(kt + 1, B1{}, std::false_type{});
    }
    if (kt < ntile) {
        tile_sync(kt);
        full_tile(kt, B0{}, std::false_type{});
    }

    if constexpr (D >= 64) {
        // after the last tile barrier the buffer without the last tile is idle
        const uint32_t stage = wave_stage(lds_addr(sm.q[ntile & 1][0]),
                                          lds_addr(sm.g[ntile & 1][0]), wave, kStageBytes<D, 1>);
        store_row_staged<D>(a.dk + goff, kw, T, lane, dk_acc, a.scale, a.gv.row, stage);
        store_row_staged<D>(a.dv + goff, kw, T, lane, dv_acc, 1.0f, a.gv.row, stage);
    } else if (kj < T) {
        store_row<D>(a.dk + goff, kj, half, dk_acc, a.scale, a.gv.row);
        store_row<D>(a.dv + goff, kj, half, dv_acc, 1.0f, a.gv.row);
    }
}

// ---------------------------------------------------------------------------------------
// The three-plane backward in the order dK/dV first, then dQ from dS.  The dK/dV stage
// already forms dS (in planes, for dK = dS^T Q); written out, it gives the dQ stage
// dQ = dS K directly, without recomputing S and dP' (two of its three products, six plane
// products each).  Before dK/dV: D = rowsum(dO o O) and the planes of dO (which the dQ
// stage wrote in the other order).
// ---------------------------------------------------------------------------------------

struct PrepArgs {
    const float *o, *dO;
    float* Dws;
    uint16_t* gp;  // dO planes out (laid out as k's)
    int BH, T;
    HeadView ov, kv;
    size_t pstride;
};

// D and the planes of dO, streaming: a thread per 8-element chunk of a row (D/8 threads per
// row, consecutive lanes), its dot product an fma chain as in chunk_dot_tree, the row's sum
// a butterfly over the chunks (xor 2, 4, ..: the pairwise tree over j of chunks 2j + half;
// then xor 1: the two halves) -- bitwise the dQ stage's D.  nrows = BH*T.
template <int D>
__global__ __launch_bounds__(256) void bwd_prep_f32x3_kernel(PrepArgs a, int nrows) {
    constexpr int kTpr = D / 8;  // threads per row
    const int gid = blockIdx.x * 256 + threadIdx.x;
    const int row = gid / kTpr;  // bh*T + t
    const int k = gid % kTpr;    // chunk
    const bool live = row < nrows;
    const int bh = live ? row / a.T : 0;
    const int t = live ? row - bh * a.T : 0;
    f32x4 g0{}, g1{}, o0{}, o1{};
    if (live) {
        const size_t off = a.ov.off(bh) + static_cast<size_t>(t) * a.ov.row + 8 * k;
        g0 = *reinterpret_cast<const f32x4*>(a.dO + off);
        g1 = *reinterpret_cast<const f32x4*>(a.dO + off + 4);
        o0 = *reinterpret_cast<const f32x4*>(a.o + off);
        o1 = *reinterpret_cast<const f32x4*>(a.o + off + 4);
    }
    float c = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) c = fmaf(g0[i], o0[i], c);
#pragma unroll
    for (int i = 0; i < 4; ++i) c = fmaf(g1[i], o1[i], c);
#pragma unroll
    for (int w = 2; w < kTpr; w *= 2) c += __shfl_xor(c, w);
    c += __shfl_xor(c, 1);
    if (!live) return;
    if (k == 0) a.Dws[row] = c;
    float x[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        x[i] = g0[i];
        x[i + 4] = g1[i];
    }
    bf16x8 pl[3];
    split_planes<3>(x, pl);
    uint16_t* dst = a.gp + a.kv.off(bh) + static_cast<size_t>(t) * a.kv.row + 8 * k;
#pragma unroll
    for (int i = 0; i < 3; ++i)
        __builtin_nontemporal_store(__builtin_bit_cast(u16x8, pl[i]),
                                    reinterpret_cast<u16x8*>(dst + i * a.pstride));
}

// Operands of the dQ-from-dS stage: k plane 0 (view kv, planes pstride apart), dS (fp32,
// layout of DkdvArgs::ds), dq fp32 out (view gv).
struct DqDsArgs {
    const uint16_t* k;
    const float* ds;
    float* dq;
    int BH, T;
    float scale;
    HeadView kv, gv;
    size_t pstride;
    int ds_n;
    int serp;  // map_block's serpentine order (set at launch)
};

// dQ^T += K^T dS^T over 32-key tiles: 128 queries per workgroup, one 32-query sub-block per
// wave.  K's planes stream through LDS in three buffers, copied two tiles ahead, and give K^T
// through transposing reads, as in the dQ stage above.  Each wave copies its 32 queries' dS
// rows of a tile (32 keys, 128 bytes each) into its own LDS slot (two slots), two tiles
// ahead, 8 lanes per row; a lane reads back the runs of its query's row that hold the 8 keys
// of a B operand (two runs of 4, in the order of the transposing reads) and splits them into
// planes, as the dK/dV stage did before writing them.  Key tiles past a wave's diagonal are
// skipped (dS is not written there);
// the diagonal tile holds the zeros of the causal mask.  All of it is asynchronous copies,
// which complete in issue order; tile kt's were issued two steps back, K's before dS's.  A
// step waits for tile kt's K copies before the barrier and for its own dS copies only after
// it, so that no wave's barrier waits for another wave's dS.
template <int D>
__global__ __launch_bounds__(kWave* kWaves) void flash_bwd_dq_ds_kernel(DqDsArgs a, int nblk) {
    constexpr int NP = 3;
    constexpr int KT = 32;             // keys per tile
    constexpr int QB = kWaves * kSub;  // queries per workgroup
    constexpr int NB = 3;              // K buffers
    using SK = Swz<D, KT>;             // a K plane tile: KT keys x D
    constexpr int kLoads = 4;  // dS copies per wave and tile: 32 rows x 128 bytes
    __shared__ __attribute__((aligned(1024))) uint16_t smk[NB][NP][SK::kBytes / 2];
    __shared__ __attribute__((aligned(1024))) float sms[kWaves][2][kLoads * 256];
    static_assert(D < 64 || 4 * kStageBytes<D, NP> <= NB * NP * SK::kBytes,
                  "four wave stages in the K buffers");
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & (kWave - 1);
    const int col = lane & 31;
    const int half = lane >> 5;
    const int T = a.T;
    int bh, blk;
    map_block(blockIdx.x, a.BH, nblk, true, a.serp != 0, bh, blk);
    const int q0 = blk * QB;
    const int qj = q0 + kSub * wave;
    const uint16_t* kh = a.k + a.kv.off(bh);
    const int krs = a.kv.row;
    const uint32_t k_lds = lds_addr(smk[0][0]);
    constexpr uint32_t kKBuf = NP * SK::kBytes;
    // copy instructions this wave issues per K tile (dma_tile: i = wave, wave + NW, ..)
    const int ncopy = NP * (wave < SK::kDma ? (SK::kDma - wave + kWaves - 1) / kWaves : 0);
    constexpr int kCopies = NP * ((SK::kDma + kWaves - 1) / kWaves);  // ncopy of wave 0
    static_assert(2 * kCopies + 2 * kLoads <= 15, "wait_vm_at_most's counts");
    auto copy_tile = [&](int kt, uint32_t buf) {
#pragma unroll
        for (int i = 0; i < NP; ++i)
            dma_tile<D, kWaves, KT>(kh + i * a.pstride, kt * KT, T, buf + i * SK::kBytes, wave,
                                    lane, krs);
    };
    const int kend = min(T, q0 + QB);
    const int ntile = (kend + KT - 1) / KT;
    uint32_t roffK[D / 16], troffK[D / 32];
    lane_offsets<D>(lane, roffK, troffK);
    // key tiles 0 .. qj/32 (the last one the diagonal); none when the wave's queries start past
    // T.  Rows qj + col < ds_n when qj < T.
    const int nmine = qj < T ? min(qj / KT + 1, ntile) : 0;
    const float* sbase = a.ds + ds_tile(bh, a.ds_n, min(qj, a.ds_n - 32) / 32, 0);
    // A slot holds the tile's 32 query rows of 32 keys (128 bytes); 16-byte chunk c of row r
    // at r*128 + 16*(c ^ ((r/2) % 8)).  Copy j: lane i fills slot bytes 1024j + 16i, row
    // 8j + i/8, so 8 lanes read one whole row and a copy one contiguous 1 KB of the tile.
    uint32_t soff[kLoads];
#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
        const int r = 8 * j + lane / 8;
        const int c = (lane % 8) ^ ((r >> 1) & 7);
        soff[j] = static_cast<uint32_t>((r * 32 + 4 * c) * 4);
    }
    const uint32_t s_lds = lds_addr(sms[wave][0]);
    constexpr uint32_t kSlot = kLoads * 1024;
    auto copy_ds = [&](int kt) {
        const float* b = sbase + static_cast<size_t>(kt) * 1024;  // tile (qj/32, kt)
#pragma unroll
        for (int j = 0; j < kLoads; ++j)
            dma_dwordx4(b, s_lds + static_cast<uint32_t>(kt & 1) * kSlot + 1024 * j, soff[j]);
    };
    copy_tile(0, k_lds);
    if (0 < nmine) copy_ds(0);
    if (1 < ntile) copy_tile(1, k_lds + kKBuf);
    if (1 < nmine) copy_ds(1);
    f32x16 acc[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) acc[dt] = f32x16{};
    // K tile kt is in buffer kb (tile kt+1 in kb1, kt+2 goes to kb2)
    uint32_t kb = k_lds, kb1 = k_lds + kKBuf, kb2 = k_lds + 2 * kKBuf;
    auto step = [&](int kt) {
        // (the counts are constants while the wave has two more tiles of its own: nmine <=
        // ntile)
        const bool steady = kt + 2 < nmine;
        // this wave's copies of K tile kt landed: outstanding may be only its dS of tile kt
        // and tile kt+1's copies ...
        if (steady && ncopy == kCopies)
            wait_vm<2 * kLoads + kCopies>();
        else if (steady)
            wait_vm<2 * kLoads>();
        else
            wait_vm_at_most((kt < nmine ? kLoads : 0) + (kt + 1 < ntile ? ncopy : 0) +
                            (kt + 1 < nmine ? kLoads : 0));
        __syncthreads();  // ... and every wave's; tile kt-1's buffer is no longer read
        if (kt + 2 < ntile) copy_tile(kt + 2, kb2);
        if (kt >= nmine) return;
        // dS of tile kt landed: outstanding may be only tile kt+1's and K tile kt+2's copies
        if (steady && ncopy == kCopies)
            wait_vm<kLoads + 2 * kCopies>();
        else if (steady)
            wait_vm<kLoads>();
        else
            wait_vm_at_most((kt + 1 < ntile ? ncopy : 0) + (kt + 1 < nmine ? kLoads : 0) +
                            (kt + 2 < ntile ? ncopy : 0));
        f32x4 x[kLoads];  // run j: keys 8j + 4*half .. +3 of row col (chunk 2j + half)
#pragma unroll
        for (int j = 0; j < kLoads; ++j)
            x[j] = lds_f32x4(s_lds + static_cast<uint32_t>(kt & 1) * kSlot + 128 * col +
                             16 * ((2 * j + half) ^ ((col >> 1) & 7)));
        bf16x8 b[2][NP];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            float v[8];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[e] = x[2 * u][e];
                v[e + 4] = x[2 * u + 1][e];
            }
            split_planes<NP>(v, b[u]);
        }
        if (kt + 2 < nmine) {
            wait_lds();  // the slot's reads are done before the copy into it starts
            copy_ds(kt + 2);
        }
        // the tile's K operands, then its products
        bf16x8 y[2][D / 32][NP];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
                for (int i = 0; i < NP; ++i)
                    y[u][dt][i] = lds_tr(troffK[dt] + kb + i * SK::kBytes + u * Swz<D>::rows(16),
                                         Swz<D>::rows(8));
            }
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt) acc[dt] = mma_planes<NP>(y[u][dt], b[u], acc[dt]);
        }
    };
    for (int kt = 0; kt < ntile; ++kt) {
        step(kt);
        const uint32_t t = kb;
        kb = kb1;
        kb1 = kb2;
        kb2 = t;
    }
    const size_t goff = a.gv.off(bh);
    if constexpr (D >= 64) {
        __syncthreads();  // every wave is past the last tile: the K buffers are idle
        const uint32_t stage =
            wave_stage(k_lds, k_lds + 2 * kStageBytes<D, NP>, wave, kStageBytes<D, NP>);
        store_row_staged<D>(a.dq + goff, qj, T, lane, acc, a.scale, a.gv.row, stage);
    } else {
        const int qi = qj + col;
        if (qi < T) store_row<D>(a.dq + goff, qi, half, acc, a.scale, a.gv.row);
    }
}

// One 32-query sub-block per wave at every shape: with the statistics as initial
// accumulators it measured faster than two sub-blocks per wave with the fold step (bf16
// B16 H16 T2048 d64 dQ 230.3 -> 217.9 us, B8 H16 T2048 122.9 -> 112.8; three planes at d = 32
// within 1%, bitwise the same).
template <int D, int NP>
void dq_dispatch(DqArgs<NP> a, hipStream_t stream) {
    const int nblk = (a.T + kWaves * kSub - 1) / (kWaves * kSub);
    const auto kernel = flash_bwd_dq_bf16_kernel<D, NP>;
    a.serp = a.BH * nblk <= resident_capacity(kernel, kWave * kWaves, 0) ? 1 : 0;
    hipLaunchKernelGGL(kernel, dim3(a.BH * nblk), dim3(kWave * kWaves), 0, stream, a, nblk);
}

template <int D, int NP>
void dkdv_dispatch(DkdvArgs<NP> a, hipStream_t stream) {
    constexpr int NW = kWaves;
    constexpr int kBlock = NW * kSub;
    const int nblk = (a.T + kBlock - 1) / kBlock;
    if constexpr (NP == 1) {
        const auto kernel = flash_bwd_dkdv_bf16_pipe_kernel<D>;
        // B16 H16 T2048 d64: G = 8, dK/dV 284 -> 277 us, its fetches beyond L2 2.7x -> 1.0x
        a.group = head_group(a.BH, nblk, resident_capacity(kernel, kWave * NW, 0));
        hipLaunchKernelGGL(kernel, dim3(a.BH * nblk), dim3(kWave * NW), 0, stream, a, nblk);
    } else if (a.ds != nullptr) {
        hipLaunchKernelGGL((flash_bwd_dkdv_bf16_kernel<D, NW, NP, true>), dim3(a.BH * nblk),
                           dim3(kWave * NW), 0, stream, a, nblk);
    } else {
        hipLaunchKernelGGL((flash_bwd_dkdv_bf16_kernel<D, NW, NP>), dim3(a.BH * nblk),
                           dim3(kWave * NW), 0, stream, a, nblk);
    }
}

}  // namespace

void launch_flash_bwd_dq_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                              const uint16_t* o, const uint16_t* dO, const float* m,
                              const float* l, uint16_t* dq, float* Dws, int BH, int T, int d,
                              float scale, const HeadView& xv, const HeadView& ov,
                              const HeadView& gv, hipStream_t stream) {
    const DqArgs<1> a{q, o, dO, k, v, m, l, dq, Dws, BH, T, scale, xv, xv, ov, gv, 0, nullptr};
    switch (d) {
        case 32: dq_dispatch<32, 1>(a, stream); break;
        case 64: dq_dispatch<64, 1>(a, stream); break;
        default: dq_dispatch<128, 1>(a, stream); break;
    }
}

void launch_flash_bwd_dkdv_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                const uint16_t* dO, const float* m, const float* l,
                                const float* Dws, uint16_t* dk, uint16_t* dv, int BH, int T,
                                int d, float scale, const HeadView& xv, const HeadView& ov,
                                const HeadView& gv, hipStream_t stream) {
    const DkdvArgs<1> a{q, dO, k, v, m, l, Dws, dk, dv, BH, T, scale, xv, ov, xv, gv, 0};
    switch (d) {
        case 32: dkdv_dispatch<32, 1>(a, stream); break;
        case 64: dkdv_dispatch<64, 1>(a, stream); break;
        default: dkdv_dispatch<128, 1>(a, stream); break;
    }
}

void launch_flash_bwd_dq_f32x3(const float* q, const HeadView& qv, const uint16_t* k,
                               const uint16_t* v, const HeadView& kv, size_t pstride,
                               uint16_t* do_planes, const float* o, const float* dO,
                               const HeadView& ov, const float* m, const float* l, float* dq,
                               const HeadView& gv, float* Dws, int BH, int T, int d,
                               float scale, hipStream_t stream) {
    const DqArgs<3> a{q,  o,     dO, k,  v,  m,  l,  dq,      Dws,
                      BH, T, scale, qv, kv, ov, gv, pstride, do_planes};
    if (d == 32)
        dq_dispatch<32, 3>(a, stream);
    else
        dq_dispatch<64, 3>(a, stream);
}

void launch_flash_bwd_dkdv_f32x3(const uint16_t* q, const uint16_t* dO, const HeadView& tv,
                                 size_t pstride, const float* k, const float* v,
                                 const HeadView& kv, const float* m, const float* l,
                                 const float* Dws, float* dk, float* dv, const HeadView& gv,
                                 int BH, int T, int d, float scale, hipStream_t stream,
                                 float* ds) {
    DkdvArgs<3> a{q, dO, k, v, m, l, Dws, dk, dv, BH, T, scale, tv, tv, kv, gv, pstride};
    if (ds != nullptr) {
        a.ds = ds;
        a.ds_n = ds_rows(T);
    }
    if (d == 32)
        dkdv_dispatch<32, 3>(a, stream);
    else
        dkdv_dispatch<64, 3>(a, stream);
}

void launch_bwd_prep_f32x3(const float* o, const float* dO, const HeadView& ov,
                           uint16_t* do_planes, const HeadView& kv, size_t pstride, float* Dws,
                           int BH, int T, int d, hipStream_t stream) {
    const PrepArgs a{o, dO, Dws, do_planes, BH, T, ov, kv, pstride};
    const int nrows = BH * T;
    const int nblk = static_cast<int>((static_cast<int64_t>(nrows) * (d / 8) + 255) / 256);
    if (d == 32)
        hipLaunchKernelGGL((bwd_prep_f32x3_kernel<32>), dim3(nblk), dim3(256), 0, stream, a,
                           nrows);
    else
        hipLaunchKernelGGL((bwd_prep_f32x3_kernel<64>), dim3(nblk), dim3(256), 0, stream, a,
                           nrows);
}

void launch_flash_bwd_dq_ds_f32x3(const uint16_t* k, const HeadView& kv, size_t pstride,
                                  const float* ds, float* dq, const HeadView& gv, int BH, int T,
                                  int d, float scale, hipStream_t stream) {
    DqDsArgs a{k, ds, dq, BH, T, scale, kv, gv, pstride, ds_rows(T), 0};
    constexpr int kBlock = kWaves * kSub;
    const int nblk = (T + kBlock - 1) / kBlock;
    const auto kernel = d == 32 ? flash_bwd_dq_ds_kernel<32> : flash_bwd_dq_ds_kernel<64>;
    a.serp = BH * nblk <= resident_capacity(kernel, kWave * kWaves, 0) ? 1 : 0;
    hipLaunchKernelGGL(kernel, dim3(BH * nblk), dim3(kWave * kWaves), 0, stream, a, nblk);
}

}  // namespace tcamd
