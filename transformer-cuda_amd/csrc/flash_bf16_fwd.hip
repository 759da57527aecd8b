// flash_bf16_fwd.hip - tiled causal attention forward on v_mfma_f32_32x32x16_bf16 with fp32
// accumulation, for bf16 operands (NP = 1) and for fp32 operands carried as NP = 3 bf16
// planes (bf16_tile.hpp: six plane products per product, fp32 output).
//
// Algorithm: the reference's tiled online-softmax forward (src/kernels/attention.cu:518-624),
// with the same statistics contract P_ij = exp(scale*q_i.k_j - m_i) / l_i.
//
// Layout of the work.  A workgroup of 4 waves (one per SIMD of a CU) owns 256 queries of one
// (b, h) head, as 8 sub-blocks of 32; wave w computes sub-blocks w and 7-w, so the causal
// work of the four waves is equal.  K and V stream through LDS in 64-key tiles (32 at
// d = 128 and for three planes; kKeyTile), double buffered and shared by the four waves;
// each K fragment read from LDS feeds the MFMAs of both sub-blocks of a wave.  Workgroups are issued heaviest query block first, with every
// block of a head on one XCD when the number of heads is a multiple of 8.
//
// Per 32-key half tile and sub-block:
//   S^T = K Q^T       4 MFMAs at d = 64; A = K rows from LDS (16-byte reads), B = Q in VGPRs
//   online softmax    lane l holds 16 scores of query l%32: 15 in-lane max/sum steps and one
//                     v_permlane32_swap; exponentials on v_exp_f32 in the log2 domain
//   O^T += V^T P^T    4 MFMAs; B = P straight from the S^T accumulator (rounded to bf16),
//                     A = V^T read from the row-major V tile with ds_read_tr16_b64, which
//                     hands each lane 4 consecutive keys of one head dimension: the two
//                     reads per MFMA carry exactly the keys the accumulator layout gives P.
// The running maximum used for the exponentials is only raised when a row's maximum grows by
// more than 2^8 (in exponent units), which leaves p <= 256 and the fp32 sums exact in form
// while skipping the O rescale on almost every tile; the true maximum is tracked beside it
// and the exported (m, l) are converted to it.
//
// Staging.  Tiles are copied HBM -> LDS with global_load_lds_dwordx4 (1 KB per wave
// instruction) into rows whose 16-byte chunks are XOR-swizzled by row, with padding after
// every 8 rows, so that both the row reads of K and the transposing reads of V hit distinct
// banks (bf16_tile.hpp).
//
// Three planes (NP = 3): K and V come from plane tensors, three plane tiles each; Q is read in
// fp32 and split in registers (its planes written out for the backward); P is split into
// planes as it leaves the softmax.  The tiles are 32 keys deep, so that the double-buffered
// planes (55 KB at d = 64) leave room for two workgroups per CU.
#include <math.h>

#include <type_traits>
#include <utility>

#include "device_common.hpp"
#include "bf16_tile.hpp"
#include "launch.hpp"
#include "sched.hpp"

namespace tcamd {
namespace {

using namespace bf16t;

// Keys per LDS tile: 64 for bf16 at d <= 64.  32 at d = 128, where double-buffered 64-key K
// and V tiles (68 KB) leave room for two workgroups per CU and 32-key ones for three, which
// the kernel's 168 VGPRs allow (config 4 forward 551 -> 499 us); 32 for three planes, whose
// double-buffered tiles then take 52.5 KB at d = 64 (three workgroups per CU) instead of 105.
template <int D, int NP>
constexpr int kKeyTile = (NP == 1 && D < 128) ? kRowTile : 32;
constexpr float kRescaleLog2 = 8.0f;  // raise the running max only beyond p = 2^8

// Folded softmax (bf16 operands, one sub-block per wave): Q is held times c = scale*log2 e
// (rounded to bf16 again, ~2^-9 relative per element) and minus the running maximum enters
// S^T as one more contraction step (its (hi, lo) terms against a ones operand), so the
// scores arrive in the log2 domain relative to the maximum and the exponentials take no
// per-element fma.  Three planes keep Q exact; two sub-blocks per wave keep the fma, whose
// registers the fold's operands would take from the third wave per SIMD.
template <int NP, int NSUB>
constexpr bool kFold = NP == 1 && NSUB == 1;

// Bytes of one K or V (plane) tile in LDS: the swizzled tile without the padding after its
// last 8-row block, which separates that block from no other row of the tile (every read
// stays inside one tile, and moving a whole tile keeps each read's banks distinct).  Three
// planes at d = 64 then take 52.5 KB per workgroup instead of 54, and three workgroups fit
// the 160 KB of LDS.
template <int D, int NP>
constexpr uint32_t kFwdTile = Swz<D, kKeyTile<D, NP>>::kBytes - Swz<D, kKeyTile<D, NP>>::kPad;

// Workgroups per CU the compiler is asked to fit in registers: three for the three-plane
// kernel at d = 64 with one sub-block per wave (168 VGPRs, no spills), which the LDS above
// then also allows.
template <int D, int NSUB, int NP>
constexpr int kFwdMinBlocks = (D == 64 && NSUB == 1 && NP == 3) ? 3 : 1;

// Double-buffered K and V tiles, NP planes each.  The row stores of Q's planes and of O go
// through LDS stages inside an idle buffer (d >= 64; at d = 32 four stages do not fit).
template <int D, int NP>
struct FwdSmem {
    uint16_t k[2][NP][kFwdTile<D, NP> / 2];
    uint16_t v[2][NP][kFwdTile<D, NP> / 2];
    static_assert(D < 64 || 2 * kStageBytes<D, NP> <= 2 * NP * kFwdTile<D, NP>,
                  "two wave stages per K (or V) array");
};
template <int D>
constexpr bool kStaged = D >= 64;
// The output's wave stages go into the buffer without the last tile when two fit there (no
// barrier needed), else into the whole K and V arrays after one more barrier.
template <int D, int NP>
constexpr bool kStageIdle = 2 * kStageBytes<D, NP> <= NP * kFwdTile<D, NP>;

// Maximum and sum of a lane's 16 scores as balanced trees (dependency depth 3 and 4 instead
// of 8 and 16 for a running reduction).
__device__ __forceinline__ float max_tree16(const f32x16& s) {
    const float a = fmaxf(fmaxf(s[0], s[1]), s[2]), b = fmaxf(fmaxf(s[3], s[4]), s[5]);
    const float c = fmaxf(fmaxf(s[6], s[7]), s[8]), d = fmaxf(fmaxf(s[9], s[10]), s[11]);
    const float e = fmaxf(fmaxf(s[12], s[13]), s[14]);
    return fmaxf(fmaxf(fmaxf(a, b), c), fmaxf(fmaxf(d, e), s[15]));
}
__device__ __forceinline__ float sum_tree16(const f32x16& s) {
    float t[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) t[i] = s[2 * i] + s[2 * i + 1];
#pragma unroll
    for (int i = 0; i < 4; ++i) t[i] += t[i + 4];
    return (t[0] + t[2]) + (t[1] + t[3]);
}

// Per-wave softmax state of one 32-query sub-block.  Folded: m_used is in log2 units of
// c*q.k, xs carries the terms of -m_used, and m_true is not kept (the exported m is m_used);
// otherwise in units of q.k.
template <int D>
struct SubState {
    f32x16 acc[D / 32];  // O^T accumulator
    float m_used;        // max the exponentials are taken against
    float m_true;        // running max of the scores (unfolded)
    float l;             // running sum of the exponentials against m_used
    bf16x8 xs;           // folded: statistic chunk of -m_used
};

// Masks S^T for keys kb.. against queries qj + col, runs the online-softmax update of `st`,
// and packs P as the two B operands (NP planes each) of the PV products.
template <int D, int NP, bool FOLD>
__device__ __forceinline__ void softmax_step(f32x16& s, SubState<D>& st, bf16x8 (&pb)[2][NP],
                                             int kb, int qj, int col, int half, float c) {
    if (kb + 31 > qj) {  // the half tile crosses the diagonal of this sub-block
#pragma unroll
        for (int r = 0; r < 16; ++r)
            if (kb + acc_row(r, half) > qj + col) s[r] = -INFINITY;
    }
    float mx = max_tree16(s);
    mx = xhalf_max(mx);
    if constexpr (FOLD) {
        // s = c*q.k - m_used already
        const bool first = st.l == 0.0f;  // l >= 1 after the first tile
        if (__builtin_amdgcn_ballot_w64(first || mx > kRescaleLog2) != 0) {
            // the first tile sets the maximum, later ones only raise it; the new offset is
            // what its bf16 terms carry
            const u16x4 t = stat_terms<NP>(-(st.m_used + (first ? mx : fmaxf(mx, 0.0f))));
            const float m_new = -(bf16_bits_to_f32(t[0]) + bf16_bits_to_f32(t[1]));
            const float shift = m_new - st.m_used;
            const float alpha = first ? 1.0f : exp2_fast(-shift);  // acc, l are 0 at first
            st.l *= alpha;
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt) st.acc[dt] *= alpha;
#pragma unroll
            for (int r = 0; r < 16; ++r) s[r] -= shift;
            st.m_used = m_new;
            u16x8 x = u16x8{};
            if (half == 0) {
                x[0] = t[0];
                x[1] = t[1];
            }
            st.xs = __builtin_bit_cast(bf16x8, x);
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] = exp2_fast(s[r]);
        st.l += xhalf_sum(sum_tree16(s));
        pack_planes<NP>(s, 0, pb[0]);
        pack_planes<NP>(s, 1, pb[1]);
        return;
    }
    st.m_true = fmaxf(st.m_true, mx);
    if (__builtin_amdgcn_ballot_w64((mx - st.m_used) * c > kRescaleLog2) != 0) {
        const float m_new = fmaxf(st.m_used, mx);
        const float alpha = exp2_fast((st.m_used - m_new) * c);  // 0 at the start
        st.l *= alpha;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) st.acc[dt] *= alpha;
        st.m_used = m_new;
    }
    const float mc = st.m_used * c;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = exp2_fast(fmaf(s[r], c, -mc));
    st.l += xhalf_sum(sum_tree16(s));
    pack_planes<NP>(s, 0, pb[0]);
    pack_planes<NP>(s, 1, pb[1]);
}

// One 32-key half tile (keys kb..kb+31, tile rows 32h..) for sub-block 1, and sub-block 0
// too when BOTH.  ka[st] / va[dt]: this lane's LDS read addresses in plane 0 of the current
// tiles for the K chunk of step st and the V^T fragment of head-dim tile dt (half 0, keys
// 0..); plane i lies i tile sizes further.
template <int D, bool BOTH, int NP, bool FOLD>
__device__ __forceinline__ void half_step(int kb, const uint32_t (&ka)[D / 16],
                                          const uint32_t (&va)[D / 32],
                                          const bf16x8 (&q0)[D / 16][NP],
                                          const bf16x8 (&q1)[D / 16][NP], SubState<D>& st0,
                                          SubState<D>& st1, int qj0, int qj1, int col, int half,
                                          float c, const bf16x8& one) {
    constexpr uint32_t kPlane = kFwdTile<D, NP>;
    f32x16 s0 = f32x16{}, s1 = f32x16{};
    if constexpr (FOLD) {  // -m_used into every score of the query
        s1 = mfma_32x32x16_bf16(one, st1.xs, s1);
        if constexpr (BOTH) s0 = mfma_32x32x16_bf16(one, st0.xs, s0);
    }
#pragma unroll
    for (int st = 0; st < D / 16; ++st) {
        bf16x8 a[NP];
#pragma unroll
        for (int i = 0; i < NP; ++i) a[i] = lds_b128(ka[st] + i * kPlane);
        s1 = mma_planes<NP>(a, q1[st], s1);
        if constexpr (BOTH) s0 = mma_planes<NP>(a, q0[st], s0);
    }
    bf16x8 p0[2][NP], p1[2][NP];
    softmax_step<D, NP, FOLD>(s1, st1, p1, kb, qj1, col, half, c);
    if constexpr (BOTH) softmax_step<D, NP, FOLD>(s0, st0, p0, kb, qj0, col, half, c);
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            bf16x8 a[NP];
#pragma unroll
            for (int i = 0; i < NP; ++i)
                a[i] = lds_tr(va[dt] + i * kPlane + u * Swz<D>::rows(16), Swz<D>::rows(8));
            st1.acc[dt] = mma_planes<NP>(a, p1[u], st1.acc[dt]);
            if constexpr (BOTH) st0.acc[dt] = mma_planes<NP>(a, p0[u], st0.acc[dt]);
        }
    }
}

// Output element type: bf16 for the bf16 path, fp32 for fp32 operands carried as planes.
template <int NP>
using OutT = std::conditional_t<NP == 1, uint16_t, float>;

// NSUB = 2: 256 queries per workgroup, wave w owns sub-blocks w (0) and 7-w (1).
// NSUB = 1: 128 queries per workgroup, wave w owns sub-block w (1) (small grids).
// k, v: plane 0 of NP bf16 planes, pstride elements apart (xv addresses a plane).  NP = 1:
// q is bf16 like k; NP = 3: Q comes from the fp32 tensor qf (view qv) and is split here,
// and its planes are written to qp (laid out as k's) when qp is not null.  serp picks the
// block order: 1 map_block's serpentine, 0 its plain order, -G heads in groups of G.
template <int D, int NSUB, int NP>
__global__ __launch_bounds__(kWave* kWaves, (kFwdMinBlocks<D, NSUB, NP>)) void flash_fwd_bf16_kernel(
    const uint16_t* __restrict__ q, const float* __restrict__ qf,
    const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, OutT<NP>* __restrict__ o,
    float* __restrict__ m_out, float* __restrict__ l_out, int BH, int T, float scale, int nblk,
    HeadView xv, HeadView qv, HeadView ov, size_t pstride, uint16_t* __restrict__ qp,
    int serp) {
    constexpr int KT = kKeyTile<D, NP>;
    constexpr int kHalves = KT / 32;  // 32-key half tiles per tile
    using S = Swz<D, KT>;
    constexpr uint32_t kBuf = NP * kFwdTile<D, NP>;  // one K (or V) buffer: NP plane tiles
    __shared__ __attribute__((aligned(1024))) FwdSmem<D, NP> sm;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int lane = threadIdx.x & (kWave - 1);
    const int col = lane & 31;
    const int half = lane >> 5;
    int bh, blk;
    if (serp < 0)
        map_block_grouped(blockIdx.x, BH, nblk, -serp, true, bh, blk);
    else
        map_block(blockIdx.x, BH, nblk, true, serp != 0, bh, blk);
    constexpr int kBlock = kWaves * NSUB * kSub;
    const int q0 = blk * kBlock;
    const int qj0 = q0 + kSub * wave;                                     // sub-block 0
    const int qj1 = NSUB == 2 ? q0 + kSub * (2 * kWaves - 1 - wave) : qj0;  // sub-block 1
    const size_t xoff = xv.off(bh), ooff = ov.off(bh);  // q, k, v head / o head
    const int xrs = xv.row, ors = ov.row;
    const uint16_t* kh = k + xoff;
    const uint16_t* vh = v + xoff;
    const float c = scale * kLog2e;

    bf16x8 qr0[D / 16][NP], qr1[D / 16][NP];
    if constexpr (NP == 1) {
        if constexpr (NSUB == 2)
            load_rowop_planes<D, NP>(qr0, q + xoff, pstride, qj0 + col, T, half, xrs);
        load_rowop_planes<D, NP>(qr1, q + xoff, pstride, qj1 + col, T, half, xrs);
        if constexpr (kFold<NP, NSUB>) {
#pragma unroll
            for (int st = 0; st < D / 16; ++st) {
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    qr1[st][0][e] = static_cast<__bf16>(static_cast<float>(qr1[st][0][e]) * c);
            }
        }
    } else {
        const float* qh = qf + qv.off(bh);
        if constexpr (NSUB == 2) load_rowop_split<D, NP>(qr0, qh, qj0 + col, T, half, qv.row);
        load_rowop_split<D, NP>(qr1, qh, qj1 + col, T, half, qv.row);
        if (qp != nullptr && !kStaged<D>) {
            if constexpr (NSUB == 2)
                store_planes<D, NP>(qp + xoff, pstride, qr0, qj0 + col, T, half);
            store_planes<D, NP>(qp + xoff, pstride, qr1, qj1 + col, T, half);
        }
    }

    const int kend = min(T, q0 + kBlock);
    const int ntile = (kend + KT - 1) / KT;
    const uint32_t k_lds = lds_addr(sm.k[0][0]);
    const uint32_t v_lds = lds_addr(sm.v[0][0]);
    // Tile kt of K and V (every plane) into buffer kt % 2.
    auto copy_tile = [&](int kt) {
        const uint32_t buf = static_cast<uint32_t>(kt & 1) * kBuf;
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            dma_tile<D, kWaves, KT>(kh + i * pstride, kt * KT, T,
                                    k_lds + buf + i * kFwdTile<D, NP>, wave, lane, xrs);
            dma_tile<D, kWaves, KT>(vh + i * pstride, kt * KT, T,
                                    v_lds + buf + i * kFwdTile<D, NP>, wave, lane, xrs);
        }
    };
    copy_tile(0);

    // Lane read offsets within a tile (K row reads, V transposing reads).
    uint32_t koff[D / 16], voff[D / 32];
    lane_offsets<D>(lane, koff, voff);

    SubState<D> st0, st1;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
        st0.acc[dt] = f32x16{};
        st1.acc[dt] = f32x16{};
    }
    st0.m_used = st1.m_used = kFold<NP, NSUB> ? 0.0f : -INFINITY;
    st0.m_true = st1.m_true = -INFINITY;
    st0.l = st1.l = 0.0f;
    st0.xs = st1.xs = bf16x8{};
    const bf16x8 one = ones_chunk<NP>(half);

    // Half tiles hh = 0 .. kHalves*ntile-1 (keys 32*hh ..).  Sub-block w is active for
    // hh < hA, sub-block 7-w for hh < hB; every wave takes part in every tile's barrier and
    // copy.  Three straight loops keep the accumulators out of any control-flow join.
    const int nhalf_t = (T + 31) / 32;
    const int hA = NSUB == 2 ? min(qj0 / 32 + 1, nhalf_t) : 0;
    const int hB = min(qj1 / 32 + 1, nhalf_t);
    const int hend = kHalves * ntile;
    uint32_t ka[D / 16], va[D / 32];
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
        for (int st = 0; st < D / 16; ++st) ka[st] = k_lds + base + koff[st];
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) va[dt] = v_lds + base + voff[dt];
    };
    int hh = 0;
    for (; hh < hA; ++hh) {
        tile_sync(hh);
        half_step<D, true, NP, kFold<NP, NSUB>>(32 * hh, ka, va, qr0, qr1, st0, st1, qj0, qj1, col, half, c, one);
    }
    for (; hh < hB; ++hh) {
        tile_sync(hh);
        half_step<D, false, NP, kFold<NP, NSUB>>(32 * hh, ka, va, qr0, qr1, st0, st1, qj0, qj1, col, half, c, one);
    }
    for (; hh < hend; ++hh) tile_sync(hh);

    // After the last tile barrier no wave reads, and no copy writes, the buffer that does not
    // hold the last tile; after one more barrier, no wave reads either buffer.
    uint32_t ostage;
    if constexpr (kStageIdle<D, NP>) {
        ostage = wave_stage(lds_addr(sm.k[ntile & 1][0]), lds_addr(sm.v[ntile & 1][0]), wave,
                            kStageBytes<D, NP>);
    } else {
        __syncthreads();
        ostage = wave_stage(lds_addr(sm.k[0][0]), lds_addr(sm.v[0][0]), wave,
                            kStageBytes<D, NP>);
    }
#pragma unroll
    for (int j = 2 - NSUB; j < 2; ++j) {
        const SubState<D>& st = j == 0 ? st0 : st1;
        const int qj = j == 0 ? qj0 : qj1;
        const int qi = qj + col;
        if constexpr (kStaged<D>) {  // whole wave; rows at or past T are not stored
            store_row_staged<D>(o + ooff, qj, T, lane, st.acc, 1.0f / st.l, ors, ostage);
            // Q's planes go out here rather than before the loop, where the first tile's
            // wait for its copies (vector-memory counts retire in order) would wait for them
            if constexpr (NP > 1)
                if (qp != nullptr)
                    store_planes_staged<D, NP>(qp + xoff, pstride, j == 0 ? qr0 : qr1, qj, T,
                                               lane, ostage);
        }
        if (qi < T) {
            if constexpr (!kStaged<D>) store_row<D>(o + ooff, qi, half, st.acc, 1.0f / st.l, ors);
            if (half == 0) {
                const size_t r = static_cast<size_t>(bh) * T + qi;
                // folded (bf16): the reference value the exponentials were taken against and
                // the sum against it; otherwise m = scale * max_j q.k, l relative to it
                if constexpr (kFold<NP, NSUB>) {
                    if (m_out != nullptr) m_out[r] = st.m_used * (1.0f / kLog2e);
                    if (l_out != nullptr) l_out[r] = st.l;
                } else {
                    if (m_out != nullptr) m_out[r] = st.m_true * scale;
                    if (l_out != nullptr)
                        l_out[r] = st.l * exp2_fast((st.m_used - st.m_true) * c);
                }
            }
        }
    }
}


template <int... Is, typename F>
__device__ __forceinline__ void static_for_impl(std::integer_sequence<int, Is...>, F&& f) {
    (f(std::integral_constant<int, Is>{}), ...);
}
// f(integral_constant<int, 0>) ... f(integral_constant<int, N-1>), in order.
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(std::make_integer_sequence<int, N>{}, f);
}

// ---------------------------------------------------------------------------------------
// The bf16 forward (NP = 1): one 32-query sub-block per wave, folded softmax, and a
// reference maximum that is set once and raised only when a row's sums grow large.
//
// On a SIMD the VALU and MFMA work of these kernels mostly add up rather than overlap
// (counters at config 3: the kernel above keeps the VALU issuing 74% of its cycles and the
// MFMA busy 46%, ~90% of the cycles one or the other), so its time follows the VALU work per
// MFMA.  Per 32-key half tile and wave it issues 9 MFMAs and about 80 VALU instructions, a
// row maximum (a max tree, a cross-half swap and a wave vote) among them.  Here the
// exponentials are taken against M, set to the row's maximum over the wave's first half tile
// and carried into the scores as their accumulators' initial value (kFwdStatInit); no
// maximum is formed after that.  Instead each
// half tile's row sum of P = 2^(s - M), which l needs anyway, is compared with 2^16: only a
// row whose scores rose more than ~11 (log2 units) above M (or an inf or NaN) makes the wave
// recompute the half tile's scores from the same LDS tile, raise M to their maximum and scale
// the accumulator and l down (raise_ref).  For unit-variance scores the maximum over 32 keys
// is within ~3 of the maximum over thousands, so the wave never takes that path there; the
// accumulated P stay below 2^11 per element as they stayed below 2^8 with the running
// maximum.  (m, l) = (M, l) honour the statistics contract P_ij = exp(scale*q_i.k_j - m_i) /
// l_i with the log-sum-exp m + ln l; m is a score of the row's first keys (or the maximum of
// a later half tile that raised it), not necessarily the row maximum.  Every LDS address of
// the unrolled loop is a lane offset plus a constant.  Per half tile at d = 64: 8 MFMAs (9
// with -M as a contraction step: config 3 forward 157.6 -> 151.6 us without it) and
// 16 v_exp_f32, 8 conversions, the 17 steps of the row sum and a compare of VALU work.
// ---------------------------------------------------------------------------------------

constexpr float kRaiseSum = 65536.0f;  // a half tile's row sum that makes M rise

// How -M enters S^T.  A lane holds one query, so M is the same in all 16 rows of its
// accumulator: with kFwdStatInit the product starts from -M (a 16-register copy per lane,
// exact in fp32), otherwise from one more contraction step, the A operand `one` times the
// (hi, lo) bf16 terms of -M (M rounded to 16 bits so that the two terms hold it exactly).
constexpr bool kFwdStatInit = true;

template <int D>
struct FoldState {
    f32x16 acc[D / 32];  // O^T
    float l;             // row sum of 2^(s - M)
    float m_used;        // M, log2 units of c*q.k
    bf16x8 xs;           // statistic chunk of -M (zero before the first half tile)
    f32x16 ms;           // kFwdStatInit: -M in every row
};

// M := m (the fold: m to 16 bits, and its (hi, lo) terms as the statistic chunk).
template <int D>
__device__ __forceinline__ void set_ref(FoldState<D>& st, float m, int half) {
    if constexpr (kFwdStatInit) {
        st.m_used = m;
#pragma unroll
        for (int r = 0; r < 16; ++r) st.ms[r] = -m;
    } else {
        const u16x4 t = stat_terms<1>(-m);
        st.m_used = -(bf16_bits_to_f32(t[0]) + bf16_bits_to_f32(t[1]));
        u16x8 x = u16x8{};
        if (half == 0) {
            x[0] = t[0];
            x[1] = t[1];
        }
        st.xs = __builtin_bit_cast(bf16x8, x);
    }
}

// S^T - M of one half tile: -M (FOLD), then K (cQ)^T over the head dimension.
template <int D, bool FOLD, bool MASK>
__device__ __forceinline__ f32x16 fold_scores(uint32_t kbase, const uint32_t (&koff)[D / 16],
                                              const bf16x8 (&qr)[D / 16], const FoldState<D>& st,
                                              int kb, int qj, int col, int half,
                                              const bf16x8& one) {
    f32x16 s = f32x16{};
    if constexpr (FOLD && kFwdStatInit) s = st.ms;
    if constexpr (FOLD && !kFwdStatInit) s = mfma_32x32x16_bf16(one, st.xs, s);
#pragma unroll
    for (int i = 0; i < D / 16; ++i) s = mfma_32x32x16_bf16(lds_b128(koff[i] + kbase), qr[i], s);
    if constexpr (MASK) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
            if (kb + acc_row(r, half) > qj + col) s[r] = -INFINITY;
    }
    return s;
}

// One half tile: K rows at kbase + koff[st], V^T at vbase + voff[dt] (LDS byte addresses).
// FIRST: the wave's first half tile, which sets M.  MASK: the half tile holds keys past some
// of the sub-block's queries.
template <int D, bool FIRST, bool MASK>
__device__ __forceinline__ void fold_half(uint32_t kbase, uint32_t vbase,
                                          const uint32_t (&koff)[D / 16],
                                          const uint32_t (&voff)[D / 32],
                                          const bf16x8 (&qr)[D / 16], FoldState<D>& st, int kb,
                                          int qj, int col, int half, const bf16x8& one) {
    f32x16 s = fold_scores<D, !FIRST, MASK>(kbase, koff, qr, st, kb, qj, col, half, one);
    if constexpr (FIRST) {
        set_ref(st, xhalf_max(max_tree16(s)), half);
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] -= st.m_used;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = exp2_fast(s[r]);
    float ts = xhalf_sum(sum_tree16(s));
    if constexpr (!FIRST) {
        if (__builtin_expect(__builtin_amdgcn_ballot_w64(!(ts < kRaiseSum)) != 0, 0)) {
            // Rare: a row's sum reached kRaiseSum (or is not finite).  The scores again from
            // the same LDS tile, M raised to their maximum where that is larger, the
            // accumulator and l scaled to the new M, and P against it.
            s = fold_scores<D, true, MASK>(kbase, koff, qr, st, kb, qj, col, half, one);
            const float mx = xhalf_max(max_tree16(s));  // relative to M
            if (mx > 0.0f) {
                const float m_old = st.m_used;
                set_ref(st, m_old + mx, half);
                const float shift = st.m_used - m_old;
                const float alpha = exp2_fast(-shift);
                st.l *= alpha;
#pragma unroll
                for (int dt = 0; dt < D / 32; ++dt) st.acc[dt] *= alpha;
#pragma unroll
                for (int r = 0; r < 16; ++r) s[r] -= shift;
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) s[r] = exp2_fast(s[r]);
            ts = xhalf_sum(sum_tree16(s));
        }
    }
    st.l += ts;
    bf16x8 pb[2];
    pb[0] = pack_b(s, 0);
    pb[1] = pack_b(s, 1);
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
        for (int u = 0; u < 2; ++u)
            st.acc[dt] = mfma_32x32x16_bf16(
                lds_tr(voff[dt] + vbase + u * Swz<D>::rows(16), Swz<D>::rows(8)), pb[u],
                st.acc[dt]);
    }
}

template <int D>
__global__ __launch_bounds__(kWave* kWaves, D >= 128 ? 3 : 4) void flash_fwd_fold_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, uint16_t* __restrict__ o, float* __restrict__ m_out,
    float* __restrict__ l_out, int BH, int T, float scale, int nblk, HeadView xv, HeadView ov,
    int serp) {
    constexpr int KT = kKeyTile<D, 1>;
    constexpr int kHalves = KT / 32;
    constexpr int kPer = 2 * kHalves;  // half tiles per round of the two buffers
    using S = Swz<D, KT>;
    constexpr uint32_t kTile = kFwdTile<D, 1>;
    __shared__ __attribute__((aligned(1024))) FwdSmem<D, 1> sm;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & (kWave - 1);
    const int col = lane & 31;
    const int half = lane >> 5;
    int bh, blk;
    if (serp < 0)
        map_block_grouped(blockIdx.x, BH, nblk, -serp, true, bh, blk);
    else
        map_block(blockIdx.x, BH, nblk, true, serp != 0, bh, blk);
    constexpr int kBlock = kWaves * kSub;
    const int q0 = blk * kBlock;
    const int qj = q0 + kSub * wave;
    const size_t xoff = xv.off(bh), ooff = ov.off(bh);
    const int xrs = xv.row;
    const uint16_t* kh = k + xoff;
    const uint16_t* vh = v + xoff;
    const float c = scale * kLog2e;

    bf16x8 qr[D / 16];  // c*Q, rounded to bf16 again
    load_rowop<D>(qr, q + xoff, qj + col, T, half, xrs);
#pragma unroll
    for (int st = 0; st < D / 16; ++st) {
#pragma unroll
        for (int e = 0; e < 8; ++e)
            qr[st][e] = static_cast<__bf16>(static_cast<float>(qr[st][e]) * c);
    }

    const int kend = min(T, q0 + kBlock);
    const int ntile = (kend + KT - 1) / KT;
    const uint32_t k_lds = lds_addr(sm.k[0][0]);
    const uint32_t v_lds = lds_addr(sm.v[0][0]);
    auto copy_tile = [&](int kt) {
        const uint32_t buf = static_cast<uint32_t>(kt & 1) * kTile;
        dma_tile<D, kWaves, KT>(kh, kt * KT, T, k_lds + buf, wave, lane, xrs);
        dma_tile<D, kWaves, KT>(vh, kt * KT, T, v_lds + buf, wave, lane, xrs);
    };
    copy_tile(0);

    uint32_t koff[D / 16], voff[D / 32];
    lane_offsets<D>(lane, koff, voff);

    FoldState<D> st;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) st.acc[dt] = f32x16{};
    st.l = 0.0f;
    st.m_used = 0.0f;
    st.xs = bf16x8{};
    const bf16x8 one = ones_chunk<1>(half);

    const int nhalf_t = (T + 31) / 32;
    const int hB = min(qj / 32 + 1, nhalf_t);  // half tiles of this wave; the last one masks
    const int hend = kHalves * ntile;
    // Tile barrier at the first half of a tile: this wave's copies of tile hh/kHalves landed,
    // every wave's too, and the other buffer is no longer read: the next tile goes there.
    auto sync_at = [&](int hh) {
        if (hh % kHalves == 0) {
            wait_vm<0>();
            __syncthreads();
            const int kt = hh / kHalves;
            if (kt + 1 < ntile) copy_tile(kt + 1);
        }
    };
    // Half tile hh with hh % kPer == P (compile time): every LDS address a constant offset.
    auto step = [&](int hh, auto Pc) {
        constexpr int P = decltype(Pc)::value;
        constexpr uint32_t base = static_cast<uint32_t>(P / kHalves) * kTile +
                                  static_cast<uint32_t>(P % kHalves) * S::rows(32);
        if constexpr (P % kHalves == 0) {
            wait_vm<0>();
            __syncthreads();
            const int kt = hh / kHalves;
            if (kt + 1 < ntile) copy_tile(kt + 1);
        }
        fold_half<D, false, false>(k_lds + base, v_lds + base, koff, voff, qr, st, 32 * hh, qj,
                                   col, half, one);
    };
    // Any half tile, its buffer and half at run time (the steps outside the unrolled loop).
    auto step_any = [&](int hh, auto first, auto mask) {
        sync_at(hh);
        const uint32_t base = static_cast<uint32_t>((hh / kHalves) & 1) * kTile +
                              static_cast<uint32_t>(hh % kHalves) * S::rows(32);
        fold_half<D, decltype(first)::value, decltype(mask)::value>(
            k_lds + base, v_lds + base, koff, voff, qr, st, 32 * hh, qj, col, half, one);
    };
    // hh = 0 sets M1 (masked when it is also the diagonal); then the unmasked half tiles,
    // kPer at a time with constant addresses; then the diagonal one.
    if (hB == 1) step_any(0, std::true_type{}, std::true_type{});
    else step_any(0, std::true_type{}, std::false_type{});
    int hh = 1;
    const int hsteady = hB - 1;
    for (; hh < hsteady && hh % kPer != 0; ++hh) step_any(hh, std::false_type{}, std::false_type{});
    for (; hh + kPer <= hsteady; hh += kPer)
        static_for<kPer>([&](auto Pc) { step(hh + decltype(Pc)::value, Pc); });
    for (; hh < hsteady; ++hh) step_any(hh, std::false_type{}, std::false_type{});
    if (hh < hB) {
        step_any(hh, std::false_type{}, std::true_type{});
        ++hh;
    }
    for (; hh < hend; ++hh) sync_at(hh);

    uint32_t ostage;
    if constexpr (kStageIdle<D, 1>) {
        ostage = wave_stage(lds_addr(sm.k[ntile & 1][0]), lds_addr(sm.v[ntile & 1][0]), wave,
                            kStageBytes<D, 1>);
    } else {
        __syncthreads();
        ostage = wave_stage(lds_addr(sm.k[0][0]), lds_addr(sm.v[0][0]), wave,
                            kStageBytes<D, 1>);
    }
    const int qi = qj + col;
    if constexpr (kStaged<D>)
        store_row_staged<D>(o + ooff, qj, T, lane, st.acc, 1.0f / st.l, ov.row, ostage);
    if (qi < T) {
        if constexpr (!kStaged<D>) store_row<D>(o + ooff, qi, half, st.acc, 1.0f / st.l, ov.row);
        if (half == 0) {
            const size_t r = static_cast<size_t>(bh) * T + qi;
            if (m_out != nullptr) m_out[r] = st.m_used * (1.0f / kLog2e);
            if (l_out != nullptr) l_out[r] = st.l;
        }
    }
}

// Operands of one forward launch.
template <int NP>
struct FwdArgs {
    const uint16_t* q;  // bf16 (NP = 1)
    const float* qf;    // fp32 (NP = 3)
    const uint16_t *k, *v;
    OutT<NP>* o;
    float *m_out, *l_out;
    int BH, T;
    float scale;
    HeadView xv, qv, ov;
    size_t pstride;
    uint16_t* qp;  // Q planes out (NP = 3), or null
};

template <int D, int NSUB, int NP>
void fwd_launch(const FwdArgs<NP>& a, hipStream_t stream) {
    constexpr int kBlock = kWaves * NSUB * kSub;
    const int nblk = (a.T + kBlock - 1) / kBlock;
    const auto kernel = flash_fwd_bf16_kernel<D, NSUB, NP>;
    // grids the device holds at once: the serpentine order (1); larger ones: heads in groups
    // (-G; B16 H16 T2048 d64: G = 16, forward 173 -> 167 us), or the plain order (0)
    const int res = resident_capacity(kernel, kWave * kWaves, 0);
    const int serp = a.BH * nblk <= res ? 1 : -head_group(a.BH, nblk, res);
    hipLaunchKernelGGL(kernel, dim3(a.BH * nblk), dim3(kWave * kWaves), 0, stream, a.q, a.qf,
                       a.k, a.v, a.o, a.m_out, a.l_out, a.BH, a.T, a.scale, nblk, a.xv, a.qv,
                       a.ov, a.pstride, a.qp, serp);
}

template <int D>
void fwd_fold_launch(const FwdArgs<1>& a, hipStream_t stream) {
    constexpr int kBlock = kWaves * kSub;
    const int nblk = (a.T + kBlock - 1) / kBlock;
    const auto kernel = flash_fwd_fold_kernel<D>;
    const int res = resident_capacity(kernel, kWave * kWaves, 0);
    const int serp = a.BH * nblk <= res ? 1 : -head_group(a.BH, nblk, res);
    hipLaunchKernelGGL(kernel, dim3(a.BH * nblk), dim3(kWave * kWaves), 0, stream, a.q, a.k,
                       a.v, a.o, a.m_out, a.l_out, a.BH, a.T, a.scale, nblk, a.xv, a.ov, serp);
}

template <int D, int NP>
void fwd_dispatch(const FwdArgs<NP>& a, hipStream_t stream) {
    if constexpr (NP == 1 && D <= 64) {
        fwd_fold_launch<D>(a, stream);
    } else if constexpr (NP == 1 || D >= 128) {
        // bf16 operands: one sub-block per wave at every size.  Its folded softmax (one
        // v_exp_f32 and no fma per score, 110 VGPRs: four waves per SIMD) outruns two
        // sub-blocks' balanced causal work (168 VGPRs, three waves): config 3 -4%,
        // T = 16384 -3%, B4 H16 T2048 -28%.  d = 128: two sub-blocks do not fit two waves.
        fwd_launch<D, 1, NP>(a, stream);
    } else if (use_single_subblock(a.BH, a.T)) {
        fwd_launch<D, 1, NP>(a, stream);
    } else {
        fwd_launch<D, 2, NP>(a, stream);
    }
}

}  // namespace

void launch_flash_fwd_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                           uint16_t* o, float* m_out, float* l_out, int BH, int T, int d,
                           float scale, const HeadView& xv, const HeadView& ov,
                           hipStream_t stream) {
    const FwdArgs<1> a{q, nullptr, k, v, o, m_out, l_out, BH, T, scale, xv, xv, ov, 0, nullptr};
    switch (d) {
        case 32: fwd_dispatch<32, 1>(a, stream); break;
        case 64: fwd_dispatch<64, 1>(a, stream); break;
        default: fwd_dispatch<128, 1>(a, stream); break;
    }
}

void launch_flash_fwd_f32x3(const float* q, const HeadView& qv, const uint16_t* k,
                            const uint16_t* v, size_t pstride, uint16_t* q_planes, float* o,
                            float* m_out, float* l_out, int BH, int T, int d, float scale,
                            const HeadView& xv, const HeadView& ov, hipStream_t stream) {
    const FwdArgs<3> a{nullptr, q,  k,  v,  o,  m_out,   l_out,
                       BH,      T,  scale, xv, qv, ov,   pstride, q_planes};
    if (d == 32)
        fwd_dispatch<32, 3>(a, stream);
    else
        fwd_dispatch<64, 3>(a, stream);
}

}  // namespace tcamd
